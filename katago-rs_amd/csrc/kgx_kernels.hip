// HIP kernels for gfx950 (CDNA4) around the convolutions: board masks, pooling, the head's small matmuls and
// spatial outputs, RMSNorm, attention and the FFN activation, on the NHWC activation layout ([batch * 361][C],
// channels contiguous), which is also the token layout of the transformer blocks.
//
// Pooling follows tools/bin2onnx/bin2onnx.py:1203-1247, RMSNorm tools/bin2onnx/bin2onnx.py:1338-1348 and
// crates/katago-nn-burn/src/tfk/kernels.rs:275-305, attention crates/katago-nn-burn/src/tfk/kernels.rs:442-613.
#include "kgx_device.h"

#include <cmath>

namespace kgx {

// ---------------------------------------------------------------------------------------------------------
// Board mask and pooling
// ---------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void mask_prep_kernel(const float* __restrict__ bin, int nin, float* __restrict__ mask,
                                                        float* __restrict__ area, float* __restrict__ s1,
                                                        float* __restrict__ s2) {
  const int b = blockIdx.x, tid = threadIdx.x;
  __shared__ float red[4];
  float sum = 0.f;
  for (int p = tid; p < HW; p += 256) {
    const float v = bin[(size_t)b * nin * HW + p];
    mask[(size_t)b * HW + p] = v;
    sum += v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if ((tid & 63) == 0) red[tid >> 6] = sum;
  __syncthreads();
  if (tid == 0) {
    const float a = (red[0] + red[1]) + (red[2] + red[3]);
    area[b] = a;
    const float c = sqrtf(a) - 14.f;
    s1[b] = c * 0.1f;
    s2[b] = c * c * 0.01f - 0.1f;
  }
}

void launch_mask_prep(const float* bin, int nin, float* mask, float* area, float* s1, float* s2, int B, hipStream_t s) {
  mask_prep_kernel<<<B, 256, 0, s>>>(bin, nin, mask, area, s1, s2);
  KGX_CHECK_LAUNCH();
}

// 64 channels x 16 groups of board points per workgroup; partial sums and maxima meet in LDS.
template <bool VALUE, bool PRO, int ACT>
__global__ __launch_bounds__(1024) void pool_kernel(const float* __restrict__ x, int ldx, int coff, int C, Prologue pro,
                                                    const float* __restrict__ area, const float* __restrict__ s1,
                                                    const float* __restrict__ s2, float* __restrict__ out) {
  const int c = blockIdx.x * 64 + threadIdx.x, b = blockIdx.y, ty = threadIdx.y;
  __shared__ float ssum[16][64], smax[16][64];
  float sum = 0.f, mx = -FLT_MAX;
  if (c < C) {
    float sc = 0.f, bi = 0.f;
    if constexpr (PRO) { sc = pro.scale[c]; bi = pro.bias[c]; }
    const float* xb = x + (size_t)b * HW * ldx + coff + c;
    const float* mb = pro.mask + (size_t)b * HW;
#pragma unroll 4
    for (int p = ty; p < HW; p += 16) {
      float v = xb[(size_t)p * ldx];
      const float mk = mb[p];
      if constexpr (PRO) v = act_f<ACT>(v * sc + bi) * mk;
      sum += v;
      if constexpr (!VALUE) mx = fmaxf(mx, v + (mk * 1e4f - 1e4f));
    }
  }
  ssum[ty][threadIdx.x] = sum;
  smax[ty][threadIdx.x] = mx;
  __syncthreads();
  if (ty == 0 && c < C) {
    float s = 0.f, m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      s += ssum[k][threadIdx.x];
      m = fmaxf(m, smax[k][threadIdx.x]);
    }
    const float mean = s / area[b];
    float* o = out + (size_t)b * 3 * C;
    o[c] = mean;
    o[C + c] = mean * s1[b];
    if constexpr (VALUE) o[2 * C + c] = mean * s2[b];
    else o[2 * C + c] = m;
  }
}

void launch_pool(const float* x, int ldx, int coff, int C, const Prologue& pro, const float* area, const float* s1,
                 const float* s2, bool value, float* out, int B, hipStream_t s) {
  dim3 grid((C + 63) / 64, B), block(64, 16);
  const bool p = pro.scale != nullptr;
#define KGX_POOL(V, P, A) pool_kernel<V, P, A><<<grid, block, 0, s>>>(x, ldx, coff, C, pro, area, s1, s2, out)
#define KGX_POOL_ACT(V)                                   \
  if (!p) KGX_POOL(V, false, ACT_ID);                     \
  else switch (pro.act) {                                 \
      case ACT_RELU: KGX_POOL(V, true, ACT_RELU); break;  \
      case ACT_MISH: KGX_POOL(V, true, ACT_MISH); break;  \
      case ACT_SILU: KGX_POOL(V, true, ACT_SILU); break;  \
      default: KGX_POOL(V, true, ACT_ID); break;          \
    }
  if (value) { KGX_POOL_ACT(true) } else { KGX_POOL_ACT(false) }
#undef KGX_POOL_ACT
#undef KGX_POOL
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Small matmuls (global inputs, pooled features, value head)
// ---------------------------------------------------------------------------------------------------------
// One batch row per workgroup: the row is staged in LDS, each thread owns one output and keeps four
// independent partial sums so that the weight loads of consecutive inputs are in flight together.

template <int ACT>
__global__ __launch_bounds__(256) void small_mm_kernel(const float* __restrict__ in, int ldin, int IC,
                                                       const float* __restrict__ W, int OC, const float* __restrict__ bias,
                                                       float* __restrict__ out, long ldout, int ostride, int accumulate) {
  extern __shared__ float xs[];
  const int b = blockIdx.y, tid = threadIdx.x;
  for (int i = tid; i < IC; i += 256) xs[i] = in[(size_t)b * ldin + i];
  __syncthreads();
  const int o = blockIdx.x * 256 + tid;
  if (o >= OC) return;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  int i = 0;
  for (; i + 4 <= IC; i += 4) {
    a0 += xs[i] * W[(size_t)i * OC + o];
    a1 += xs[i + 1] * W[(size_t)(i + 1) * OC + o];
    a2 += xs[i + 2] * W[(size_t)(i + 2) * OC + o];
    a3 += xs[i + 3] * W[(size_t)(i + 3) * OC + o];
  }
  for (; i < IC; i++) a0 += xs[i] * W[(size_t)i * OC + o];
  float acc = (a0 + a1) + (a2 + a3);
  if (bias) acc += bias[o];
  acc = act_f<ACT>(acc);
  float* p = out + (size_t)b * ldout + (size_t)o * ostride;
  *p = accumulate ? *p + acc : acc;
}

void launch_small_matmul(const float* in, int ldin, int IC, const float* W, int OC, const float* bias, int act,
                         float* out, long ldout, int ostride, bool accumulate, int B, hipStream_t s) {
  if (IC > 16384) throw std::runtime_error("small_matmul: input too wide");
  dim3 grid((OC + 255) / 256, B);
  const size_t lds = (size_t)IC * sizeof(float);
  const int a = accumulate ? 1 : 0;
  switch (act) {
    case ACT_RELU: small_mm_kernel<ACT_RELU><<<grid, 256, lds, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
    case ACT_MISH: small_mm_kernel<ACT_MISH><<<grid, 256, lds, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
    case ACT_SILU: small_mm_kernel<ACT_SILU><<<grid, 256, lds, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
    default: small_mm_kernel<ACT_ID><<<grid, 256, lds, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
  }
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Head: policy p2 conv and ownership conv per board point, written into the readback rows
// ---------------------------------------------------------------------------------------------------------
// 64 board points per workgroup; their rows of H are staged in LDS with coalesced loads first.

template <int PACT, int VACT>
__global__ __launch_bounds__(64) void head_spatial_kernel(HeadSpatialArgs a) {
  extern __shared__ float hs[];
  const int b = blockIdx.y, p0 = blockIdx.x * 64, tid = threadIdx.x;
  const int np = min(64, HW - p0);
  const float* src = a.H + ((size_t)b * HW + p0) * a.ldh;
  for (int e = tid; e < np * a.ldh; e += 64) hs[e] = src[e];
  __syncthreads();
  const int pos = p0 + tid;
  if (tid >= np) return;
  const float* h = hs + (size_t)tid * a.ldh;
  const float mk = a.mask[(size_t)b * HW + pos];
  float pol[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < a.c_p1; c++) {
    const float v = act_f<PACT>((h[a.p1_off + c] + a.p1_bias[(size_t)b * a.c_p1 + c]) * a.p1_scale[c] + a.p1_shift[c]) * mk;
#pragma unroll
    for (int p = 0; p < 4; p++)
      if (p < a.P) pol[p] += v * a.w_p2[c * a.P + p];
  }
  float own = 0.f;
  for (int c = 0; c < a.c_v1; c++) {
    const float v = act_f<VACT>(h[a.v1_off + c] * a.v1_scale[c] + a.v1_shift[c]) * mk;
    own += v * a.w_own[c];
  }
  float* row = a.out + (size_t)b * a.row_len;
#pragma unroll
  for (int p = 0; p < 4; p++)
    if (p < a.P) row[p * (HW + 1) + pos] = pol[p];
  row[a.own_off + pos] = own;
}

void launch_head_spatial(const HeadSpatialArgs& a, int B, hipStream_t s) {
  if (a.P > 4) throw std::runtime_error("head: more than 4 policy channels");
  if (a.ldh > 256) throw std::runtime_error("head: too many head channels");
  dim3 grid((HW + 63) / 64, B);
  const size_t lds = (size_t)64 * a.ldh * sizeof(float);
  if (a.p1_act != a.v1_act) throw std::runtime_error("head: p1 and v1 activations differ");
  switch (a.p1_act) {
    case ACT_RELU: head_spatial_kernel<ACT_RELU, ACT_RELU><<<grid, 64, lds, s>>>(a); break;
    case ACT_MISH: head_spatial_kernel<ACT_MISH, ACT_MISH><<<grid, 64, lds, s>>>(a); break;
    case ACT_SILU: head_spatial_kernel<ACT_SILU, ACT_SILU><<<grid, 64, lds, s>>>(a); break;
    default: head_spatial_kernel<ACT_ID, ACT_ID><<<grid, 64, lds, s>>>(a); break;
  }
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// RMSNorm
// ---------------------------------------------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_tok_kernel(const float* __restrict__ x, int ldx, int C,
                                                          const float* __restrict__ w, float eps,
                                                          const float* __restrict__ mask, T* __restrict__ out, int ldo,
                                                          int rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + (size_t)row * ldx;
  float ss = 0.f;
  for (int c = lane; c < C; c += 64) ss += xr[c] * xr[c];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float rs = 1.f / sqrtf(ss / (float)C + eps);
  const float mk = mask[row];
  T* o = out + (size_t)row * ldo;
  for (int c = lane; c < C; c += 64) o[c] = to_t<T>(xr[c] * rs * w[c] * mk);
}

void launch_rmsnorm_tok(int prec, const float* x, int ldx, int C, const float* w, float eps, const float* mask,
                        void* out, int ldo, int rows, hipStream_t s) {
  dim3 grid((rows + 3) / 4);
  if (prec == PREC_F16) rmsnorm_tok_kernel<f16><<<grid, 256, 0, s>>>(x, ldx, C, w, eps, mask, (f16*)out, ldo, rows);
  else if (prec == PREC_BF16) rmsnorm_tok_kernel<bf16><<<grid, 256, 0, s>>>(x, ldx, C, w, eps, mask, (bf16*)out, ldo, rows);
  else rmsnorm_tok_kernel<float><<<grid, 256, 0, s>>>(x, ldx, C, w, eps, mask, (float*)out, ldo, rows);
  KGX_CHECK_LAUNCH();
}

// Spatial trunk-tip statistic: rs[b] = 1 / sqrt(sum(x^2 * mask) / (area * C) + eps).
__global__ __launch_bounds__(256) void tip_rms_stats_kernel(const float* __restrict__ x, int C,
                                                            const float* __restrict__ mask,
                                                            const float* __restrict__ area, float eps,
                                                            float* __restrict__ rs) {
  const int b = blockIdx.x, tid = threadIdx.x;
  __shared__ float red[4];
  float ss = 0.f;
  for (size_t k = tid; k < (size_t)HW * C; k += 256) {
    const size_t p = k / C;
    const float v = x[(size_t)b * HW * C + k];
    ss += v * v * mask[(size_t)b * HW + p];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  if (tid == 0) rs[b] = 1.f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (area[b] * (float)C) + eps);
}

template <int ACT>
__global__ __launch_bounds__(256) void tip_rms_apply_kernel(const float* __restrict__ x, int C,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, float eps, int spatial,
                                                            const float* __restrict__ mask,
                                                            const float* __restrict__ rs_b, float* __restrict__ out,
                                                            int rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + (size_t)row * C;
  float rs;
  if (spatial) {
    rs = rs_b[row / HW];
  } else {
    float ss = 0.f;
    for (int c = lane; c < C; c += 64) ss += xr[c] * xr[c];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    rs = 1.f / sqrtf(ss / (float)C + eps);
  }
  const float mk = mask[row];
  for (int c = lane; c < C; c += 64) out[(size_t)row * C + c] = act_f<ACT>(xr[c] * rs * gamma[c] + beta[c]) * mk;
}

void launch_tip_rms(const float* x, int C, const float* gamma, const float* beta, float eps, bool spatial, int act,
                    const float* mask, const float* area, float* rs_tmp, float* out, int B, hipStream_t s) {
  if (spatial) tip_rms_stats_kernel<<<B, 256, 0, s>>>(x, C, mask, area, eps, rs_tmp);
  const int rows = B * HW;
  dim3 grid((rows + 3) / 4);
  const int sp = spatial ? 1 : 0;
  switch (act) {
    case ACT_RELU: tip_rms_apply_kernel<ACT_RELU><<<grid, 256, 0, s>>>(x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
    case ACT_MISH: tip_rms_apply_kernel<ACT_MISH><<<grid, 256, 0, s>>>(x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
    case ACT_SILU: tip_rms_apply_kernel<ACT_SILU><<<grid, 256, 0, s>>>(x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
    default: tip_rms_apply_kernel<ACT_ID><<<grid, 256, 0, s>>>(x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
  }
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Attention: one thread per query, keys and values staged 32 at a time in LDS, online softmax
// ---------------------------------------------------------------------------------------------------------

template <typename T, int D, bool ROPE>
__global__ __launch_bounds__(64) void attn_kernel(AttnArgs a) {
  const int qi = blockIdx.x * 64 + threadIdx.x, h = blockIdx.y, n = blockIdx.z, tid = threadIdx.x;
  const int kvh = h / (a.H / a.KV);
  constexpr int HALF = D / 2;
  const bool in_range = qi < HW;
  const int qrow = in_range ? qi : 0;
  const T* qkv = (const T*)a.qkv;
  float q[D], acc[D];
  {
    const T* qp = qkv + ((size_t)n * HW + qrow) * a.ldq + a.q_off + h * D;
    if constexpr (ROPE) {
      const int tab = a.q_tables == 1 ? 0 : kvh;  // query head h uses its kv head's table
      const float* ct = a.cos_t + ((size_t)tab * HW + qrow) * HALF;
      const float* st = a.sin_t + ((size_t)tab * HW + qrow) * HALF;
#pragma unroll
      for (int p = 0; p < HALF; p++) {
        const float x0 = (float)qp[p], x1 = (float)qp[p + HALF];
        q[p] = (x0 * ct[p] - x1 * st[p]) * a.scale;
        q[p + HALF] = (x0 * st[p] + x1 * ct[p]) * a.scale;
      }
    } else {
#pragma unroll
      for (int d = 0; d < D; d++) q[d] = (float)qp[d] * a.scale;
    }
  }
#pragma unroll
  for (int d = 0; d < D; d++) acc[d] = 0.f;
  float m_run = -FLT_MAX, l_run = 0.f;
  __shared__ float ks[32 * D], vs[32 * D], kb[32];
  const int ktab = a.k_tables == 1 ? 0 : kvh;
  for (int j0 = 0; j0 < HW; j0 += 32) {
    const int cnt = min(32, HW - j0);
    for (int e = tid; e < 32 * D; e += 64) {
      const int j = e / D, d = e - j * D;
      float kv = 0.f, vv = 0.f;
      if (j < cnt) {
        const T* row = qkv + ((size_t)n * HW + j0 + j) * a.ldq;
        const T* kp = row + a.k_off + kvh * D;
        if constexpr (ROPE) {
          const int p = d < HALF ? d : d - HALF;
          const float x0 = (float)kp[p], x1 = (float)kp[p + HALF];
          const float c = a.cos_t[((size_t)ktab * HW + j0 + j) * HALF + p];
          const float sn = a.sin_t[((size_t)ktab * HW + j0 + j) * HALF + p];
          kv = d < HALF ? x0 * c - x1 * sn : x0 * sn + x1 * c;
        } else {
          kv = (float)kp[d];
        }
        vv = (float)row[a.v_off + kvh * D + d];
      }
      ks[e] = kv;
      vs[e] = vv;
    }
    if (tid < 32) kb[tid] = tid < cnt ? a.mask[(size_t)n * HW + j0 + tid] * 3e4f - 3e4f : 0.f;
    __syncthreads();
    float sc[32];
    float m_blk = m_run;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      if (j < cnt) {
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < D; d++) s += q[d] * ks[j * D + d];
        s += kb[j];
        sc[j] = s;
        m_blk = fmaxf(m_blk, s);
      }
    }
    const float alpha = __expf(m_run - m_blk);
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < D; d++) acc[d] *= alpha;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      if (j < cnt) {
        const float p = __expf(sc[j] - m_blk);
        l_run += p;
#pragma unroll
        for (int d = 0; d < D; d++) acc[d] += p * vs[j * D + d];
      }
    }
    m_run = m_blk;
    __syncthreads();
  }
  if (in_range) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    T* o = (T*)a.out + ((size_t)n * HW + qi) * a.ldo + h * D;
#pragma unroll
    for (int d = 0; d < D; d++) o[d] = to_t<T>(acc[d] * inv);
  }
}

template <typename T, int D>
static void attn_d(const AttnArgs& a, int B, hipStream_t s) {
  dim3 grid((HW + 63) / 64, a.H, B);
  if (a.q_tables > 0) attn_kernel<T, D, true><<<grid, 64, 0, s>>>(a);
  else attn_kernel<T, D, false><<<grid, 64, 0, s>>>(a);
}

template <typename T>
static void attn_t(const AttnArgs& a, int B, hipStream_t s) {
  if (a.dq != a.dv) throw std::runtime_error("attention: dq != dv unsupported");
  switch (a.dq) {
    case 16: attn_d<T, 16>(a, B, s); break;
    case 32: attn_d<T, 32>(a, B, s); break;
    case 64: attn_d<T, 64>(a, B, s); break;
    default: throw std::runtime_error("attention: head dim must be 16, 32 or 64");
  }
}

void launch_attention(int prec, const AttnArgs& a, int B, hipStream_t s) {
  if (prec == PREC_F16) attn_t<f16>(a, B, s);
  else if (prec == PREC_BF16) attn_t<bf16>(a, B, s);
  else attn_t<float>(a, B, s);
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// FFN activation
// ---------------------------------------------------------------------------------------------------------

template <typename T, bool GATED>
__global__ __launch_bounds__(256) void ffn_act_kernel(const float* __restrict__ u, int ldu, int F, T* __restrict__ h,
                                                      int ldh, int rows) {
  const size_t k = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= (size_t)rows * F) return;
  const size_t r = k / F, f = k - r * F;
  const float a = u[r * ldu + f];
  float v;
  if constexpr (GATED) v = act_f<ACT_SILU>(a) * u[r * ldu + F + f];
  else v = act_f<ACT_MISH>(a);
  h[r * ldh + f] = to_t<T>(v);
}

void launch_ffn_act(int prec, const float* u, int ldu, int F, bool gated, void* h, int ldh, int rows, hipStream_t s) {
  const size_t total = (size_t)rows * F;
  dim3 grid((unsigned)((total + 255) / 256));
#define KGX_FFN(T) \
  if (gated) ffn_act_kernel<T, true><<<grid, 256, 0, s>>>(u, ldu, F, (T*)h, ldh, rows); \
  else ffn_act_kernel<T, false><<<grid, 256, 0, s>>>(u, ldu, F, (T*)h, ldh, rows);
  if (prec == PREC_F16) { KGX_FFN(f16) }
  else if (prec == PREC_BF16) { KGX_FFN(bf16) }
  else { KGX_FFN(float) }
#undef KGX_FFN
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
