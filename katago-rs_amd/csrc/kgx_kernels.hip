// HIP kernels for gfx950 (CDNA4) around the convolutions: board masks, pooling, the head's small matmuls and
// spatial outputs, RMSNorm, attention and the FFN activation, on the NHWC activation layout ([batch * 361][C],
// channels contiguous), which is also the token layout of the transformer blocks.
//
// Pooling follows tools/bin2onnx/bin2onnx.py:1203-1247, RMSNorm tools/bin2onnx/bin2onnx.py:1338-1348 and
// crates/katago-nn-burn/src/tfk/kernels.rs:275-305, attention crates/katago-nn-burn/src/tfk/kernels.rs:442-613.
#include "kgx_device.h"

#include <cmath>
#include <map>
#include <mutex>

namespace kgx {

// The workspace of the allocation-free forward pass (kg_run_static): one static device array per GPU. Host code
// never uses the array's name as an address: static_scratch() looks up each device's copy once, with that device
// current, and every launch takes that pointer.
// The array is initialized data (one nonzero byte), not a zero-fill section, so that this code object's size in
// memory equals its size in the file: a zero-fill section at file offset 0x400 with 64 MiB extends the ELF's
// section extent 64 MiB past its bytes, and a tool that copies a loaded code object by that extent reads past the
// library's mapping. The offload bundle of this file is compressed (the Makefile), so the library stays small. The
// forward pass writes or clears every byte it reads here, so the initial contents do not matter.
static __device__ __align__(256) char scratch[kStaticScratchBytes] = {1};

void* static_scratch(int device) {
  static std::mutex mu;
  static std::map<int, void*> ptrs;
  std::lock_guard<std::mutex> lock(mu);
  auto it = ptrs.find(device);
  if (it != ptrs.end()) return it->second;
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (cur != device) throw std::runtime_error("internal: static scratch looked up on another device");
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  ptrs.emplace(device, p);
  return p;
}

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
  launch_k(mask_prep_kernel, B, 256, 0, s, bin, nin, mask, area, s1, s2);
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
#define KGX_POOL(V, P, A) launch_k(pool_kernel<V, P, A>, grid, block, 0, s, x, ldx, coff, C, pro, area, s1, s2, out)
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
// A workgroup computes 64 outputs for 8 batch rows: the rows are staged in LDS, the 4 waves take every fourth
// input (so each thread has many independent weight loads in flight, coalesced across the wave's 64 outputs) and
// their partial sums meet in LDS. Latency, not arithmetic, bounds these products; the split keeps each thread's
// dependent chain short.

template <int ACT>
__global__ __launch_bounds__(256) void small_mm_kernel(const float* __restrict__ in, int ldin, int IC,
                                                       const float* __restrict__ W, int OC, const float* __restrict__ bias,
                                                       float* __restrict__ out, long ldout, int ostride, int accumulate,
                                                       int B) {
  extern __shared__ float xs[];  // [8][IC], then [4][8][64] partial sums
  const int tid = threadIdx.x, lane = tid & 63, kg = tid >> 6;
  const int o = blockIdx.x * 64 + lane, b0 = blockIdx.y * 8;
  const int nb = min(8, B - b0);
  for (int e = tid; e < 8 * IC; e += 256) {
    const int r = e / IC, i = e - r * IC;
    xs[e] = r < nb ? in[(size_t)(b0 + r) * ldin + i] : 0.f;
  }
  __syncthreads();
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (o < OC) {
#pragma unroll 8
    for (int i = kg; i < IC; i += 4) {
      const float w = W[(size_t)i * OC + o];
#pragma unroll
      for (int r = 0; r < 8; r++) acc[r] += xs[r * IC + i] * w;
    }
  }
  float* ps = xs + 8 * IC;
#pragma unroll
  for (int r = 0; r < 8; r++) ps[(kg * 8 + r) * 64 + lane] = acc[r];
  __syncthreads();
  for (int e = tid; e < 8 * 64; e += 256) {
    const int r = e >> 6, c = e & 63, oo = blockIdx.x * 64 + c;
    if (r >= nb || oo >= OC) continue;
    float v = (ps[(0 * 8 + r) * 64 + c] + ps[(1 * 8 + r) * 64 + c]) + (ps[(2 * 8 + r) * 64 + c] + ps[(3 * 8 + r) * 64 + c]);
    if (bias) v += bias[oo];
    v = act_f<ACT>(v);
    float* p = out + (size_t)(b0 + r) * ldout + (size_t)oo * ostride;
    *p = accumulate ? *p + v : v;
  }
}

void launch_small_matmul(const float* in, int ldin, int IC, const float* W, int OC, const float* bias, int act,
                         float* out, long ldout, int ostride, bool accumulate, int B, hipStream_t s) {
  if (IC > 4096) throw std::runtime_error("small_matmul: input too wide");
  dim3 grid((OC + 63) / 64, (B + 7) / 8);
  const size_t lds = ((size_t)8 * IC + 4 * 8 * 64) * sizeof(float);
  const int a = accumulate ? 1 : 0;
  switch (act) {
    case ACT_RELU: launch_k(small_mm_kernel<ACT_RELU>, grid, 256, lds, s, in, ldin, IC, W, OC, bias, out, ldout, ostride, a, B); break;
    case ACT_MISH: launch_k(small_mm_kernel<ACT_MISH>, grid, 256, lds, s, in, ldin, IC, W, OC, bias, out, ldout, ostride, a, B); break;
    case ACT_SILU: launch_k(small_mm_kernel<ACT_SILU>, grid, 256, lds, s, in, ldin, IC, W, OC, bias, out, ldout, ostride, a, B); break;
    default: launch_k(small_mm_kernel<ACT_ID>, grid, 256, lds, s, in, ldin, IC, W, OC, bias, out, ldout, ostride, a, B); break;
  }
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Row programs: pooling and small matmuls of one batch row in one workgroup
// ---------------------------------------------------------------------------------------------------------
// The row's work is a few hundred KB of reads and tens of thousands of multiply-adds: latency, not bandwidth or
// arithmetic, bounds it, so one launch does all of it with 1024 threads, and every stage issues all of its loads
// before using any (one round trip per stage).
// Pooling: four channels per thread (16-byte loads), C/4 threads per board point, so one wave covers 64 / (C/4)
// points per load and each thread loads all of its (at most RP_PPT) points at once. Per-thread partial sums and
// maxima are combined over the lanes of a wave that share channels, then over the waves in LDS (the pooling of
// launch_pool). The row's mask is staged in LDS first.
// Matmul: each wave takes a chunk of 64 outputs (weight loads coalesced across them) and a slice of the inputs;
// partial sums meet in LDS. A program with a single matmul may split its outputs over gridDim.y workgroups per
// row, so that each streams only its share of the weights. Weights that fit are staged in LDS at the start, all
// loads of all staged matrices in flight together, so that a chain of small matmuls waits for memory once.
constexpr int RP_NT = 1024, RP_PPT = 6;  // chunks of <= 64 channels: at least 64 point slots, 6 passes cover 361

// Channels [c0, c0 + C) of one pooling, C <= 64.
__device__ void row_pool_chunk(const RowProg& P, const RowPool& q, int c0, int C, int b, float* feat, float* red,
                               const float* mk) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tpp = C / 4, pslots = RP_NT / tpp;  // threads per point, point slots per pass of all threads
  const int cg4 = tid % tpp, slot = tid / tpp, c = c0 + 4 * cg4;
  const float* xb = q.x + (size_t)b * HW * q.ldx + q.coff + c;
  floatx4 v[RP_PPT];
#pragma unroll
  for (int k = 0; k < RP_PPT; k++) {
    const int p = slot + pslots * k;
    v[k] = p < HW ? *(const floatx4*)(xb + (size_t)p * q.ldx) : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  floatx4 sc = {1.f, 1.f, 1.f, 1.f}, bi = {0.f, 0.f, 0.f, 0.f};
  if (q.scale) {
    sc = *(const floatx4*)(q.scale + c);
    bi = *(const floatx4*)(q.bias + c);
  }
  // Every global load of the stage is issued before its first barrier (a load after one costs a round trip).
  const float area = P.area[b], s1 = P.s1[b], s2 = P.s2[b];
  __syncthreads();  // the staged mask
  floatx4 sum = {0.f, 0.f, 0.f, 0.f}, mx = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
  auto accum = [&](auto actc) {  // straight-line per activation (no switch inside the unrolled loop)
    constexpr int A = decltype(actc)::value;
#pragma unroll
    for (int k = 0; k < RP_PPT; k++) {
      const int p = slot + pslots * k;
      if (p < HW) {
        const float m = mk[p], pen = m * 1e4f - 1e4f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float x = v[k][e];
          if (A >= 0) x = act_f<A < 0 ? ACT_ID : A>(x * sc[e] + bi[e]) * m;
          sum[e] += x;
          mx[e] = fmaxf(mx[e], x + pen);
        }
      }
    }
  };
  if (!q.scale) accum(std::integral_constant<int, -1>{});
  else if (q.act == ACT_RELU) accum(std::integral_constant<int, ACT_RELU>{});
  else if (q.act == ACT_MISH) accum(std::integral_constant<int, ACT_MISH>{});
  else if (q.act == ACT_SILU) accum(std::integral_constant<int, ACT_SILU>{});
  else accum(std::integral_constant<int, ACT_ID>{});
  // Lanes l and l ^ (tpp << j) of a wave hold the same channels.
  for (int off = tpp; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      sum[e] += __shfl_xor(sum[e], off);
      mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], off));
    }
  }
  if (lane < tpp) {
    *(floatx4*)(red + wave * C + 4 * cg4) = sum;
    *(floatx4*)(red + RP_NT + wave * C + 4 * cg4) = mx;
  }
  __syncthreads();
  if (tid < C) {
    float s = 0.f, m = -FLT_MAX;
    for (int w = 0; w < RP_NT / 64; w++) {
      s += red[w * C + tid];
      m = fmaxf(m, red[RP_NT + w * C + tid]);
    }
    const float mean = s / area;
    feat[c0 + tid] = mean;
    feat[q.C + c0 + tid] = mean * s1;
    feat[2 * q.C + c0 + tid] = q.value ? mean * s2 : m;
  }
  __syncthreads();
}

__device__ void row_pool(const RowProg& P, const RowPool& q, int b, float* feat, float* red, const float* mk) {
  for (int c0 = 0; c0 < q.C; c0 += 64) row_pool_chunk(P, q, c0, min(64, q.C - c0), b, feat, red, mk);
}

// Outputs [o_begin, o_end) of one matmul for row b.
__device__ void row_mm(const RowMM& m, int b, float* lds, float* red, int o_begin, int o_end) {
  constexpr int NW = RP_NT / 64, KB = 16;  // waves, loads in flight per batch
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const float* gin = m.gin ? m.gin + (size_t)b * m.ldgin : nullptr;
  const float* lin = lds + m.src;
  const int nch = (o_end - o_begin + 63) / 64;
  for (int ch0 = 0; ch0 < nch; ch0 += NW) {
    const int nc = min(NW, nch - ch0), nks = NW / nc;  // chunks this round, K slices per chunk
    const int ch = ch0 + w % nc, ks = w / nc;
    const int o = o_begin + ch * 64 + lane;
    const bool fin = w < nc && o < o_end;  // this thread finishes output o
    // Every global load of the stage is issued before its first barrier (a load after one costs a round trip).
    const float bo = fin && m.bias ? (m.bias_lds ? lds[m.wlds + m.IC * m.OC + o] : m.bias[o]) : 0.f;
    float* op = fin && m.out ? m.out + (size_t)b * m.ldout + (size_t)o * m.ostride : nullptr;
    const float prev = op && m.accumulate ? *op : 0.f;
    float acc = 0.f;
    if (ks < nks && o < o_end) {
      const bool slice = m.wlds >= 0 && m.wcols > 0;
      const float* wcol = slice ? lds + m.wlds + (o - o_begin) : (m.wlds >= 0 ? lds + m.wlds : m.W) + o;
      const int wst = slice ? m.wcols : m.OC;
      for (int i0 = ks; i0 < m.IC; i0 += KB * nks) {
        float wv[KB], xv[KB];
#pragma unroll
        for (int j = 0; j < KB; j++) {
          const int i = i0 + j * nks;
          wv[j] = i < m.IC ? wcol[(size_t)i * wst] : 0.f;
          xv[j] = i < m.IC ? (gin ? gin[i] : lin[i]) : 0.f;
        }
        // Explicit fused multiply-adds, as in the gpool tile kernel's matmul, which gives the same bits: the
        // compiler's contraction of a multiply and an add may differ between the two loops.
#pragma unroll
        for (int j = 0; j < KB; j++) acc = __builtin_fmaf(xv[j], wv[j], acc);
      }
    }
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (fin) {
      float v = 0.f;
      for (int k = 0; k < nks; k++) v += red[(k * nc + w) * 64 + lane];
      v = act_rt(v + bo, m.act);
      if (m.dst >= 0) lds[m.dst + o] = v;
      if (op) *op = prev + v;
    }
    __syncthreads();
  }
}

// One row program for row b; with nsplit > 1 this workgroup computes share `split` of the last matmul's outputs.
__device__ void run_row_prog(const RowProg& P, int b, int split, int nsplit, float* lds) {
  // [lds_floats] features, intermediates and staged weights, [2 RP_NT] reduction scratch, [HW] the row's mask
  float* red = lds + P.lds_floats;
  float* mk = red + 2 * RP_NT;
  if (P.npool > 0)
    for (int p = threadIdx.x; p < HW; p += RP_NT) mk[p] = P.mask[(size_t)b * HW + p];
  // Pooling from the producer's partials (RowPool::part, first pooling only): this thread's channel's sums and
  // maxima of the row's tiles (at most three), loaded with the program's first loads.
  const RowPool* pq = P.npool > 0 && P.pool[0].psum ? &P.pool[0] : nullptr;
  long long pps[3] = {0, 0, 0};
  float ppm[3] = {-FLT_MAX, -FLT_MAX, -FLT_MAX};
  if (pq && (int)threadIdx.x < pq->C) {
    const int t0 = b * HW / pq->ppt, t1 = (b * HW + HW - 1) / pq->ppt;
#pragma unroll
    for (int j = 0; j < 3; j++) {
      const int t = t0 + j;
      if (t <= t1) {
        const size_t at = (size_t)(t * 2 + (t * pq->ppt / HW == b ? 0 : 1)) * pq->C + threadIdx.x;
        pps[j] = pq->psum[at];
        ppm[j] = pq->pmax[at];
      }
    }
  }
  // The emission's inputs come first: this thread's x vectors into registers, the share's batch-norm scale and
  // bias into LDS after the mask (the barrier after the weight staging publishes them).
  const RowEmit& E = P.emit;
  floatx4 ex[RE_MAX][2];
  int e_o0 = 0, e_n8 = 0;
  float* esb = mk + HW;
  if (E.x) {
    const int per = P.mm[P.nmm - 1].OC / nsplit;
    e_o0 = split * per;
    e_n8 = per / 8;
#pragma unroll
    for (int k = 0; k < RE_MAX; k++) {
      const int v = threadIdx.x + k * RP_NT;
      if (v < HW * e_n8) {
        const int p = v / e_n8, c = e_o0 + (v - p * e_n8) * 8;
        const float* xp = E.x + ((size_t)b * HW + p) * E.ldx + c;
        ex[k][0] = *(const floatx4*)xp;
        ex[k][1] = *(const floatx4*)(xp + 4);
      }
    }
    for (int i = threadIdx.x; i < 2 * per; i += RP_NT) esb[i] = i < per ? E.scale[e_o0 + i] : E.bias[e_o0 + i - per];
  }
  {
    // Staged weights: the whole set as one list of 16-byte vectors, RP_WB loads per thread in flight. A matmul
    // staged as a column share (wcols) contributes the IC rows of its wcols columns from this split's first one.
    constexpr int RP_WB = 8;
    int total = 0;
    for (int k = 0; k < P.nmm; k++) total += P.mm[k].w4;
    for (int v0 = 0; v0 < total; v0 += RP_NT * RP_WB) {
      floatx4 buf[RP_WB];
      float* dst[RP_WB];
#pragma unroll
      for (int j = 0; j < RP_WB; j++) {
        int v = v0 + j * RP_NT + threadIdx.x, k = 0;
        dst[j] = nullptr;
        if (v < total) {
          for (; k < P.nmm; k++) {
            const int n4 = P.mm[k].w4;
            if (v < n4) break;
            v -= n4;
          }
          const RowMM& m = P.mm[k];
          if (m.wcols > 0) {
            const int q4 = m.wcols / 4, i = v / q4, c = (v - i * q4) * 4;
            buf[j] = *(const floatx4*)(m.W + (size_t)i * m.OC + split * m.wcols + c);
          } else {
            buf[j] = *(const floatx4*)(m.W + 4 * v);  // (with bias_lds, the bias follows W in memory)
          }
          dst[j] = lds + m.wlds + 4 * v;
        }
      }
#pragma unroll
      for (int j = 0; j < RP_WB; j++)
        if (dst[j]) *(floatx4*)dst[j] = buf[j];
    }
    __syncthreads();
  }
  for (int k = 0; k < P.npool; k++) {
    if (k == 0 && pq) {
      if ((int)threadIdx.x < pq->C) {
        const float s = (float)((double)(pps[0] + pps[1] + pps[2]) / (double)kPoolFix);
        const float m = fmaxf(fmaxf(ppm[0], ppm[1]), ppm[2]);
        const float mean = s / P.area[b];
        float* feat = lds + pq->dst;
        feat[threadIdx.x] = mean;
        feat[pq->C + threadIdx.x] = mean * P.s1[b];
        feat[2 * pq->C + threadIdx.x] = pq->value ? mean * P.s2[b] : m;
      }
      __syncthreads();
    } else {
      row_pool(P, P.pool[k], b, lds + P.pool[k].dst, red, mk);
    }
  }
  for (int k = 0; k < P.nmm; k++) {
    const RowMM& m = P.mm[k];
    int o0 = 0, o1 = m.OC;
    if (k == P.nmm - 1 && nsplit > 1) {
      const int per = (m.OC + nsplit - 1) / nsplit;
      o0 = min(m.OC, split * per);
      o1 = min(m.OC, o0 + per);
    }
    row_mm(m, b, lds, red, o0, o1);
  }
  if (E.x) {
    // row_mm ends with a barrier: the share's per-row bias is in LDS at the last matmul's dst.
    const float* rb = lds + P.mm[P.nmm - 1].dst;
    const int per = e_n8 * 8;
#pragma unroll
    for (int k = 0; k < RE_MAX; k++) {
      const int v = threadIdx.x + k * RP_NT;
      if (v < HW * e_n8) {
        const int p = v / e_n8, cl = (v - p * e_n8) * 8, c = e_o0 + cl;
        const float m = mk[p];
        // One activation branch per vector (not per value: the program runs once per workgroup, from a cold
        // instruction cache).
        float t[8];
#pragma unroll
        for (int e = 0; e < 8; e++) t[e] = (ex[k][e >> 2][e & 3] + rb[c + e]) * esb[cl + e] + esb[per + cl + e];
        switch (E.act) {
          case ACT_RELU:
#pragma unroll
            for (int e = 0; e < 8; e++) t[e] = act_f<ACT_RELU>(t[e]) * m;
            break;
          case ACT_MISH:  // (16-bit outputs in act16's form)
            if (E.prec != PREC_F32) {
#pragma unroll
              for (int e = 0; e < 8; e++) t[e] = act16<ACT_MISH>(t[e], m);
            } else {
#pragma unroll
              for (int e = 0; e < 8; e++) t[e] = act_f<ACT_MISH>(t[e]) * m;
            }
            break;
          case ACT_SILU:
#pragma unroll
            for (int e = 0; e < 8; e++) t[e] = act_f<ACT_SILU>(t[e]) * m;
            break;
          default:
#pragma unroll
            for (int e = 0; e < 8; e++) t[e] *= m;
        }
        u32x4 w;
        if (E.prec == PREC_F16) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const f16 l = to_t<f16>(t[2 * e]), h = to_t<f16>(t[2 * e + 1]);
            w[e] = __builtin_bit_cast(unsigned short, l) | ((unsigned)__builtin_bit_cast(unsigned short, h) << 16);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const bf16 l = to_t<bf16>(t[2 * e]), h = to_t<bf16>(t[2 * e + 1]);
            w[e] = __builtin_bit_cast(unsigned short, l) | ((unsigned)__builtin_bit_cast(unsigned short, h) << 16);
          }
        }
        *(u32x4*)((unsigned short*)E.out + ((size_t)b * HW + p) * E.ldo + c) = w;
      }
    }
  }
}

// blockIdx.x: the batch row; blockIdx.y: the program (several independent programs), or the output share of the
// single program's last matmul.
__global__ __launch_bounds__(RP_NT) void row_prog_kernel(RowProgs PS) {
  extern __shared__ float lds[];
  // One call site, so that the program's code is in the kernel once.
  const bool several = PS.n > 1;
  run_row_prog(PS.p[several ? blockIdx.y : 0], blockIdx.x, several ? 0 : blockIdx.y, several ? 1 : gridDim.y, lds);
}

bool row_emit_fits(int OC, int splits) {
  return splits >= 1 && OC % splits == 0 && (OC / splits) % 8 == 0 && (OC / splits) / 8 * HW <= RE_MAX * RP_NT;
}

static size_t row_prog_check(const RowProg& p) {
  const RowEmit& e = p.emit;
  const size_t lds = ((size_t)p.lds_floats + 2 * RP_NT + HW + (e.x ? 2 * p.mm[p.nmm > 0 ? p.nmm - 1 : 0].OC : 0)) *
                     sizeof(float);
  if (e.x) {
    const RowMM& lm = p.mm[p.nmm > 0 ? p.nmm - 1 : 0];
    if (p.nmm < 1 || p.npool < 1 || lm.dst < 0 || lm.dst + lm.OC > p.lds_floats || !row_emit_fits(lm.OC, p.splits) ||
        (e.prec != PREC_F16 && e.prec != PREC_BF16) || e.ldx % 4 || e.ldo % 8 || !e.scale || !e.bias || !e.out ||
        ((uintptr_t)e.x | (uintptr_t)e.out) % 16)
      throw std::runtime_error("row program: unsupported emission layout");
  }
  for (int k = 0; k < p.nmm; k++) {
    const RowMM& m = p.mm[k];
    // (A staged bias's copy is padded to 16 bytes, as in memory.)
    const int cols = m.wcols > 0 ? m.wcols : m.OC;
    const int n = m.bias_lds ? ((m.IC + 1) * cols + 3) / 4 * 4 : m.IC * cols;
    if (m.wlds >= 0 ? n % 4 || m.wlds % 4 || m.wlds + n > p.lds_floats || m.w4 != n / 4 : m.w4 != 0 || m.bias_lds)
      throw std::runtime_error("row program: bad staged weight layout");
    if (m.bias_lds && (m.wcols > 0 || m.bias != m.W + (size_t)m.IC * m.OC))
      throw std::runtime_error("row program: a staged bias must follow its whole W");
    // A column share is this workgroup's split of the (only) matmul's outputs, in 16-byte columns.
    if (m.wcols > 0 && (m.wlds < 0 || m.wcols % 4 || m.OC % p.splits || m.wcols != m.OC / p.splits))
      throw std::runtime_error("row program: bad staged weight share");
  }
  if (lds > 64 * 1024) throw std::runtime_error("row program: too much LDS");
  if (p.splits < 1 || (p.splits > 1 && p.nmm != 1))
    throw std::runtime_error("row program: output splits need exactly one matmul");
  for (int k = 0; k < p.npool; k++) {
    const RowPool& q = p.pool[k];
    // From partials: the first pooling only, a thread per channel, at most three tiles per row.
    if (q.psum) {
      if (k != 0 || !q.pmax || q.C > RP_NT || q.ppt * 2 < HW - 1)
        throw std::runtime_error("row program: unsupported pooling partials");
      continue;
    }
    // Pooled in chunks of 64 channels: every chunk's C/4 threads per point must divide 64 (16-byte loads).
    const int last = q.C % 64 ? q.C % 64 : 64;
    if (q.C < 4 || last % 4 || 64 % (last / 4) || q.ldx % 4 || q.coff % 4)
      throw std::runtime_error("row program: unsupported pooled channel count or layout");
  }
  return lds;
}

void launch_row_progs(const RowProgs& ps, int B, hipStream_t s) {
  if (ps.n < 1 || ps.n > RowProgs::MAX) throw std::runtime_error("row programs: bad count");
  size_t lds = 0;
  for (int k = 0; k < ps.n; k++) lds = std::max(lds, row_prog_check(ps.p[k]));
  if (ps.n > 1)
    for (int k = 0; k < ps.n; k++)
      if (ps.p[k].splits != 1) throw std::runtime_error("row programs: output splits need a single program");
  launch_k(row_prog_kernel, dim3(B, ps.n > 1 ? ps.n : ps.p[0].splits), RP_NT, lds, s, ps);
  KGX_CHECK_LAUNCH();
}

void row_prog_stage_weights(RowProg& p, size_t max_bytes) {
  int off = (p.lds_floats + 3) / 4 * 4;
  for (int k = 0; k < p.nmm; k++) {
    RowMM& m = p.mm[k];
    // A bias stored right after W in memory (padded to 16 bytes there) is staged with it, so the matmul waits on
    // no load.
    const bool fold = m.bias && m.bias == m.W + (size_t)m.IC * m.OC;
    const int n = fold ? ((m.IC + 1) * m.OC + 3) / 4 * 4 : m.IC * m.OC;
    if (n % 4 == 0 && ((size_t)off + n + 2 * RP_NT + HW) * sizeof(float) <= max_bytes) {
      m.wlds = off;
      m.bias_lds = fold;
      m.w4 = n / 4;
      off += n;
    }
  }
  p.lds_floats = off;
}

void launch_row_prog(const RowProg& p, int B, hipStream_t s) {
  RowProgs ps;
  ps.p[0] = p;
  ps.n = 1;
  launch_row_progs(ps, B, s);
}

// ---------------------------------------------------------------------------------------------------------
// Global-pooling block's mid activation per 192-pixel tile (GpoolTile)
// ---------------------------------------------------------------------------------------------------------
constexpr int GT_NT = 256, GT_BM = kGpoolTileRows, GT_KS = 16, GT_RV = 4, GT_RW = 12;

int gpool_tile_share(int cg, int cr) {
  const int share = cr / 8;
  return cr % 64 == 0 && share <= 40 && 3 * cg >= 64 && 3 * cg <= 384 && 3 * cg * share <= 4 * GT_RW * GT_NT ? share
                                                                                                        : 0;
}

template <typename T, int ACT>
__global__ __launch_bounds__(GT_NT) void gpool_tile_kernel(GpoolTile a, int M) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, SH = a.share, IC = 3 * a.cg, cg = a.cg;
  int t, sh;
  gpool_tile_of(blockIdx.x, a.cr / SH, t, sh);
  const int c0 = sh * SH;
  const int m0 = t * GT_BM;
  if (m0 >= M) {
    l2_touch_keep(l2_touch(a.pf, a.pf_bytes, tid));
    return;
  }
  const int b0 = m0 / HW, nrow = (min(m0 + GT_BM, M) - 1) / HW - b0 + 1;  // batch rows touched: 1 or 2
  // LDS: W share [IC][SH], features [2][IC], matmul slices [2][GT_KS][SH], row biases [2][SH], scale and bias
  // [2][SH], mask [GT_BM].
  float* const wl = lds;
  float* const feat = wl + IC * SH;
  float* const part = feat + 2 * IC;
  float* const rb = part + 2 * GT_KS * SH;
  float* const esb = rb + 2 * SH;
  float* const mk = esb + 2 * SH;
  // Every load first: this thread's x vectors (8 channels each), the pooled partials of (row, channel), the mask,
  // the weight share and the batch-norm share.
  const int n8 = SH / 8, nv = GT_BM * n8;
  floatx4 ex[GT_RV][2];
#pragma unroll
  for (int k = 0; k < GT_RV; k++) {
    const int v = tid + k * GT_NT, p = v / n8, m = min(m0 + p, M - 1);
    if (v < nv) {
      const float* xp = a.x + (size_t)m * a.ldx + c0 + (v - p * n8) * 8;
      ex[k][0] = *(const floatx4*)xp;
      ex[k][1] = *(const floatx4*)(xp + 4);
    }
  }
  const int pr = tid / cg, pc = tid - pr * cg;
  long long pps[3] = {0, 0, 0};
  float ppm[3] = {-FLT_MAX, -FLT_MAX, -FLT_MAX}, area = 1.f, s1 = 0.f;
  if (pr < nrow) {
    const int b = b0 + pr, t0 = b * HW / GT_BM, t1 = (b * HW + HW - 1) / GT_BM;
#pragma unroll
    for (int q = 0; q < 3; q++) {
      const int tq = t0 + q;
      if (tq <= t1) {
        const size_t at = (size_t)(tq * 2 + (tq * GT_BM / HW == b ? 0 : 1)) * cg + pc;
        pps[q] = a.psum[at];
        ppm[q] = a.pmax[at];
      }
    }
    area = a.area[b];
    s1 = a.s1[b];
  }
  const float mkv = tid < GT_BM && m0 + tid < M ? a.mask[m0 + tid] : 0.f;
  const int w4 = IC * SH / 4, q4 = SH / 4;
  floatx4 wr[GT_RW];
#pragma unroll
  for (int k = 0; k < GT_RW; k++) {
    const int v = tid + k * GT_NT;
    if (v < w4) {
      const int i = v / q4;
      wr[k] = *(const floatx4*)(a.W + (size_t)i * a.cr + c0 + (v - i * q4) * 4);
    }
  }
  const float esv = tid < 2 * SH ? (tid < SH ? a.scale[c0 + tid] : a.bias[c0 + tid - SH]) : 0.f;
#pragma unroll
  for (int k = 0; k < GT_RW; k++) {
    const int v = tid + k * GT_NT;
    if (v < w4) *(floatx4*)(wl + 4 * v) = wr[k];
  }
  if (tid < GT_BM) mk[tid] = mkv;
  if (tid < 2 * SH) esb[tid] = esv;
  // The row's pooled features (as the row program forms them from partials).
  if (pr < nrow) {
    const float sum = (float)((double)(pps[0] + pps[1] + pps[2]) / (double)kPoolFix);
    const float mx = fmaxf(fmaxf(ppm[0], ppm[1]), ppm[2]);
    const float mean = sum / area;
    feat[pr * IC + pc] = mean;
    feat[pr * IC + cg + pc] = mean * s1;
    feat[pr * IC + 2 * cg + pc] = mx;
  }
  __syncthreads();
  // The matmul: slice ks of output o of row r sums inputs ks, ks + 16, ... in order; the row bias then sums the
  // slices in order (row_mm's order with one 64-output chunk over 16 waves).
  for (int task = tid; task < nrow * SH * GT_KS; task += GT_NT) {
    const int r = task / (SH * GT_KS), rem = task - r * SH * GT_KS, ks = rem / SH, o = rem - ks * SH;
    const float* fr = feat + r * IC;
    const float* wo = wl + o;
    float acc = 0.f;
    // Four inputs' LDS reads issued before their four multiply-adds (in input order), so that a thread waits for
    // LDS once per four inputs instead of once per input.
    int i = ks;
    for (; i + 3 * GT_KS < IC; i += 4 * GT_KS) {
      float f[4], w[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f[j] = fr[i + j * GT_KS];
        w[j] = wo[(i + j * GT_KS) * SH];
      }
#pragma unroll
      for (int j = 0; j < 4; j++) acc = __builtin_fmaf(f[j], w[j], acc);  // (fused, as in row_mm)
    }
    for (; i < IC; i += GT_KS) acc = __builtin_fmaf(fr[i], wo[i * SH], acc);
    part[(r * GT_KS + ks) * SH + o] = acc;
  }
  __syncthreads();
  if (tid < nrow * SH) {
    const int r = tid / SH, o = tid - r * SH;
    float v = 0.f;
    for (int k = 0; k < GT_KS; k++) v += part[(r * GT_KS + k) * SH + o];
    rb[r * SH + o] = act_rt(v + 0.f, ACT_ID);
  }
  __syncthreads();
  const int pfv = l2_touch(a.pf, a.pf_bytes, tid);
#pragma unroll
  for (int k = 0; k < GT_RV; k++) {
    const int v = tid + k * GT_NT, p = v / n8, m = m0 + p;
    if (v < nv && m < M) {
      const int cl = (v - p * n8) * 8, r = m / HW - b0;
      const float mm = mk[p];
      float tv[8];
#pragma unroll
      for (int e = 0; e < 8; e++) tv[e] = (ex[k][e >> 2][e & 3] + rb[r * SH + cl + e]) * esb[cl + e] + esb[SH + cl + e];
#pragma unroll
      for (int e = 0; e < 8; e++) tv[e] = ACT == ACT_ID ? tv[e] * mm : act16<ACT>(tv[e], mm);
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const T l = to_t<T>(tv[2 * e]), h = to_t<T>(tv[2 * e + 1]);
        w[e] = __builtin_bit_cast(unsigned short, l) | ((unsigned)__builtin_bit_cast(unsigned short, h) << 16);
      }
      *(u32x4*)((unsigned short*)a.out + (size_t)m * a.ldo + c0 + cl) = w;
    }
  }
  l2_touch_keep(pfv);
}

void launch_gpool_tile(const GpoolTile& a, int B, hipStream_t s) {
  const int M = B * HW;
  if (M <= 0) return;
  if (a.share != gpool_tile_share(a.cg, a.cr) || !a.share || !a.psum || !a.pmax || !a.area || !a.s1 || !a.W ||
      !a.x || !a.scale || !a.bias || !a.mask || !a.out || a.ldx % 4 || a.ldo % 8 || a.x == nullptr ||
      ((uintptr_t)a.x | (uintptr_t)a.out | (uintptr_t)a.W) % 16 || (a.prec != PREC_F16 && a.prec != PREC_BF16))
    throw std::runtime_error("gpool tile: unsupported layout");
  const int IC = 3 * a.cg;
  const size_t lds = ((size_t)IC * a.share + 2 * IC + 2 * GT_KS * a.share + 4 * a.share + GT_BM) * sizeof(float);
  const dim3 grid(gpool_tile_grid(M, a.cr / a.share));
  auto go = [&](auto t, auto act) {
    launch_k(gpool_tile_kernel<decltype(t), decltype(act)::value>, grid, GT_NT, lds, s, a, M);
  };
  auto by_act = [&](auto t) {
    switch (a.act) {
      case ACT_RELU: go(t, std::integral_constant<int, ACT_RELU>{}); break;
      case ACT_MISH: go(t, std::integral_constant<int, ACT_MISH>{}); break;
      case ACT_SILU: go(t, std::integral_constant<int, ACT_SILU>{}); break;
      default: go(t, std::integral_constant<int, ACT_ID>{}); break;
    }
  };
  if (a.prec == PREC_F16) by_act(f16());
  else by_act(bf16());
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Head: policy p2 conv and ownership conv per board point, written into the readback rows
// ---------------------------------------------------------------------------------------------------------
// Sixteen lanes per board point: lane l of a point takes channels l, l + 16, ... of p1 and of v1 (at most 16 HK of
// each), so the point's 16 lanes read contiguous 64-byte runs of its row of H, and each lane keeps the parameters of
// its channels (this row's gpool bias, the batch norms, p2 and ownership weights) in registers for every point it
// visits. Partial sums are added over the 16 lanes. HS_PTS points of one batch row per workgroup.
constexpr int HS_PTS = 48;

template <int ACT, int HK>
__global__ __launch_bounds__(256) void head_spatial_kernel(HeadSpatialArgs a) {
  const int b = blockIdx.y, tid = threadIdx.x, l16 = tid & 15, slot = tid >> 4;
  float pb[HK], ps[HK], pt[HK], w2[HK][4], vs[HK], vt[HK], wo[HK];
#pragma unroll
  for (int k = 0; k < HK; k++) {
    const int c = l16 + 16 * k;
    const bool okp = c < a.c_p1, okv = c < a.c_v1;
    pb[k] = okp ? a.p1_bias[(size_t)b * a.c_p1 + c] : 0.f;
    ps[k] = okp ? a.p1_scale[c] : 0.f;
    pt[k] = okp ? a.p1_shift[c] : 0.f;
#pragma unroll
    for (int p = 0; p < 4; p++) w2[k][p] = (okp && p < a.P) ? a.w_p2[c * a.P + p] : 0.f;
    vs[k] = okv ? a.v1_scale[c] : 0.f;
    vt[k] = okv ? a.v1_shift[c] : 0.f;
    wo[k] = okv ? a.w_own[c] : 0.f;
  }
  // The slot's HS_PTS / 16 points: every load of all of them first (clamped points, no branch around a load), so that
  // the thread waits for memory once, then the sums; points past the row compute on the clamped copy and store nothing.
  constexpr int NP = HS_PTS / 16;
  const int p_end = min(HW, ((int)blockIdx.x + 1) * HS_PTS);
  float hp[NP][HK], hv[NP][HK], mkp[NP];
#pragma unroll
  for (int i = 0; i < NP; i++) {
    const int pos = min(blockIdx.x * HS_PTS + slot + 16 * i, p_end - 1);
    const float* h = a.H + ((size_t)b * HW + pos) * a.ldh;
    mkp[i] = a.mask[(size_t)b * HW + pos];
#pragma unroll
    for (int k = 0; k < HK; k++) {
      const int c = l16 + 16 * k;
      hp[i][k] = h[a.p1_off + min(c, a.c_p1 - 1)];
      hv[i][k] = h[a.v1_off + min(c, a.c_v1 - 1)];
    }
  }
#pragma unroll
  for (int i = 0; i < NP; i++) {
    const int pos = blockIdx.x * HS_PTS + slot + 16 * i;
    const float mk = mkp[i];
    float pol[4] = {0.f, 0.f, 0.f, 0.f}, own = 0.f;
#pragma unroll
    for (int k = 0; k < HK; k++) {
      const int c = l16 + 16 * k;
      if (c < a.c_p1) {
        const float v = act_f<ACT>((hp[i][k] + pb[k]) * ps[k] + pt[k]) * mk;
#pragma unroll
        for (int p = 0; p < 4; p++) pol[p] += v * w2[k][p];
      }
      if (c < a.c_v1) own += act_f<ACT>(hv[i][k] * vs[k] + vt[k]) * mk * wo[k];
    }
    // The 16 lanes of a point run every step alike, so the exchanges stay within active lanes.
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
#pragma unroll
      for (int p = 0; p < 4; p++) pol[p] += __shfl_xor(pol[p], off);
      own += __shfl_xor(own, off);
    }
    if (l16 == 0 && pos < p_end) {
      float* row = a.out + (size_t)b * a.row_len;
#pragma unroll
      for (int p = 0; p < 4; p++)
        if (p < a.P) row[p * (HW + 1) + pos] = pol[p];
      row[a.own_off + pos] = own;
    }
  }
}

template <int HK>
static void head_spatial_launch(const HeadSpatialArgs& a, int B, hipStream_t s) {
  dim3 grid((HW + HS_PTS - 1) / HS_PTS, B);
  switch (a.p1_act) {
    case ACT_RELU: launch_k(head_spatial_kernel<ACT_RELU, HK>, grid, 256, 0, s, a); break;
    case ACT_MISH: launch_k(head_spatial_kernel<ACT_MISH, HK>, grid, 256, 0, s, a); break;
    case ACT_SILU: launch_k(head_spatial_kernel<ACT_SILU, HK>, grid, 256, 0, s, a); break;
    default: launch_k(head_spatial_kernel<ACT_ID, HK>, grid, 256, 0, s, a); break;
  }
}

void launch_head_spatial(const HeadSpatialArgs& a, int B, hipStream_t s) {
  if (a.P > 4) throw std::runtime_error("head: more than 4 policy channels");
  if (a.p1_act != a.v1_act) throw std::runtime_error("head: p1 and v1 activations differ");
  if (a.c_p1 < 1 || a.c_v1 < 1) throw std::runtime_error("head: no p1 or v1 channels");  // (the loads clamp to them)
  const int c = std::max(a.c_p1, a.c_v1);
  if (c <= 32) head_spatial_launch<2>(a, B, s);
  else if (c <= 64) head_spatial_launch<4>(a, B, s);
  else if (c <= 128) head_spatial_launch<8>(a, B, s);
  else throw std::runtime_error("head: more than 128 p1 or v1 channels");
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Readback
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void readback_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                       size_t n) {
  const size_t n4 = n / 4, step = (size_t)gridDim.x * 256;
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n4; i += step)
    ((floatx4*)dst)[i] = ((const floatx4*)src)[i];
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) dst[4 * n4 + threadIdx.x] = src[4 * n4 + threadIdx.x];
  __threadfence_system();
}

void launch_readback(const float* src, float* host_dst, size_t n, hipStream_t s) {
  if (n == 0) return;
  if (((uintptr_t)src | (uintptr_t)host_dst) % 16) throw std::runtime_error("readback: pointers not 16-byte aligned");
  const size_t blocks = std::min<size_t>((n / 4 + 255) / 256 + 1, 1024);
  launch_k(readback_kernel, dim3((unsigned)blocks), 256, 0, s, src, host_dst, n);
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

// Vector form: a row is spread over LPR lanes (a power of two with C = 8 NV LPR, so no lane idles: C = 384 takes
// 16 lanes of 24 channels, 512 takes 64 lanes of 8), each lane holding NV vectors of eight consecutive channels
// (vector j of lane l covers channels 8 (j LPR + l), so a row's lanes read 32 LPR contiguous bytes per vector). A
// wave covers 64 / LPR rows per pass and PASSES passes; every load of x and of the gains is issued before the first
// reduction, which runs over the LPR lanes of the row (log2 LPR shuffles).
template <typename T, int NV, int LPR>
__global__ __launch_bounds__(256) void rmsnorm_lanes_kernel(const float* __restrict__ x, int ldx, int C,
                                                            const float* __restrict__ w, float eps,
                                                            const float* __restrict__ mask, T* __restrict__ out,
                                                            int ldo, int rows, int region) {
  // Two passes (row groups per lane group) when a pass covers at most two rows of a wave, else one: two to four rows
  // per wave (C = 512 at 64 lanes per row is slower at four rows per wave than at two).
  constexpr int lpr = LPR, rg = 64 / LPR, PASSES = rg <= 2 ? 2 : 1, PER_WG = 4 * rg * PASSES;
  const int lane = threadIdx.x & 63, g = lane / lpr, l = lane - g * lpr;
  const int row0 = rmsnorm_first_row(blockIdx.x, region, PER_WG) + (threadIdx.x >> 6) * rg * PASSES + g;
  floatx4 v[PASSES][NV][2], wv[NV][2];
#pragma unroll
  for (int p = 0; p < PASSES; p++) {
    const float* xr = x + (size_t)min(row0 + p * rg, rows - 1) * ldx;
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const int c = (j * lpr + l) * 8;
      v[p][j][0] = *(const floatx4*)(xr + c);
      v[p][j][1] = *(const floatx4*)(xr + c + 4);
    }
  }
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int c = (j * lpr + l) * 8;
    wv[j][0] = *(const floatx4*)(w + c);
    wv[j][1] = *(const floatx4*)(w + c + 4);
  }
#pragma unroll
  for (int p = 0; p < PASSES; p++) {
    const int row = row0 + p * rg;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++)
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int e = 0; e < 4; e++) ss += v[p][j][h][e] * v[p][j][h][e];
#pragma unroll
    for (int off = lpr >> 1; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if (row >= rows) continue;
    const float rs = 1.f / sqrtf(ss / (float)C + eps), mk = mask[row];
    T* op = out + (size_t)row * ldo;
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const int c = (j * lpr + l) * 8;
      const floatx4 a = v[p][j][0] * rs * wv[j][0] * mk, b = v[p][j][1] * rs * wv[j][1] * mk;
      store4<T>(op + c, a[0], a[1], a[2], a[3]);
      store4<T>(op + c + 4, b[0], b[1], b[2], b[3]);
    }
  }
}

template <typename T, int NV, int LPR>
static void rmsnorm_lanes(const float* x, int ldx, int C, const float* w, float eps, const float* mask, T* out, int ldo,
                          int rows, hipStream_t s, int region) {
  constexpr int rg = 64 / LPR, per_wg = 4 * rg * (rg <= 2 ? 2 : 1);
  if (region % per_wg) region = 0;  // (a tile that is not whole workgroups: consecutive rows)
  launch_k(rmsnorm_lanes_kernel<T, NV, LPR>, rmsnorm_grid(rows, region, per_wg), 256, 0, s, x, ldx, C, w, eps, mask, out,
           ldo, rows, region);
}

template <typename T, int LPR>
static bool rmsnorm_nv(int nv, const float* x, int ldx, int C, const float* w, float eps, const float* mask, T* out,
                       int ldo, int rows, hipStream_t s, int region) {
  switch (nv) {
    case 1: rmsnorm_lanes<T, 1, LPR>(x, ldx, C, w, eps, mask, out, ldo, rows, s, region); return true;
    case 2: rmsnorm_lanes<T, 2, LPR>(x, ldx, C, w, eps, mask, out, ldo, rows, s, region); return true;
    case 3: rmsnorm_lanes<T, 3, LPR>(x, ldx, C, w, eps, mask, out, ldo, rows, s, region); return true;
    case 4: rmsnorm_lanes<T, 4, LPR>(x, ldx, C, w, eps, mask, out, ldo, rows, s, region); return true;
    default: return false;
  }
}

int rmsnorm_rows_per_workgroup(int C) {
  const int v8 = C / 8;
  if (C % 8 || v8 < 1) return 0;
  int lpr = 64;
  while (lpr > 4 && v8 % lpr) lpr >>= 1;
  if (v8 % lpr || v8 / lpr > 4) return 0;
  const int rg = 64 / lpr;
  return 4 * rg * (rg <= 2 ? 2 : 1);
}

// The lane layout of a row of C channels: LPR = the largest power of two up to 64 dividing C / 8, NV = C / (8 LPR);
// layouts with more than four vectors per lane take the scalar kernel.
template <typename T>
static bool rmsnorm_vec(const float* x, int ldx, int C, const float* w, float eps, const float* mask, T* out, int ldo,
                        int rows, hipStream_t s, int region) {
  const int v8 = C / 8;
  int lpr = 64;
  while (lpr > 4 && v8 % lpr) lpr >>= 1;
  if (v8 % lpr) return false;
  const int nv = v8 / lpr;
  switch (lpr) {
    case 64: return rmsnorm_nv<T, 64>(nv, x, ldx, C, w, eps, mask, out, ldo, rows, s, region);
    case 32: return rmsnorm_nv<T, 32>(nv, x, ldx, C, w, eps, mask, out, ldo, rows, s, region);
    case 16: return rmsnorm_nv<T, 16>(nv, x, ldx, C, w, eps, mask, out, ldo, rows, s, region);
    case 8: return rmsnorm_nv<T, 8>(nv, x, ldx, C, w, eps, mask, out, ldo, rows, s, region);
    default: return rmsnorm_nv<T, 4>(nv, x, ldx, C, w, eps, mask, out, ldo, rows, s, region);
  }
}

void launch_rmsnorm_tok(int prec, const float* x, int ldx, int C, const float* w, float eps, const float* mask,
                        void* out, int ldo, int rows, hipStream_t s, int region) {
  const int tsz = prec == PREC_F32 ? 4 : 2;
  if (rows > 0 && C % 8 == 0 && ldx % 4 == 0 && ldo % (16 / tsz) == 0 &&
      ((uintptr_t)x | (uintptr_t)w) % 16 == 0 && (uintptr_t)out % 16 == 0) {
    bool done;
    if (prec == PREC_F16) done = rmsnorm_vec<f16>(x, ldx, C, w, eps, mask, (f16*)out, ldo, rows, s, region);
    else if (prec == PREC_BF16) done = rmsnorm_vec<bf16>(x, ldx, C, w, eps, mask, (bf16*)out, ldo, rows, s, region);
    else done = rmsnorm_vec<float>(x, ldx, C, w, eps, mask, (float*)out, ldo, rows, s, region);
    if (done) {
      KGX_CHECK_LAUNCH();
      return;
    }
  }
  dim3 grid((rows + 3) / 4);
  if (prec == PREC_F16) launch_k(rmsnorm_tok_kernel<f16>, grid, 256, 0, s, x, ldx, C, w, eps, mask, (f16*)out, ldo, rows);
  else if (prec == PREC_BF16) launch_k(rmsnorm_tok_kernel<bf16>, grid, 256, 0, s, x, ldx, C, w, eps, mask, (bf16*)out, ldo, rows);
  else launch_k(rmsnorm_tok_kernel<float>, grid, 256, 0, s, x, ldx, C, w, eps, mask, (float*)out, ldo, rows);
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
  if (spatial) launch_k(tip_rms_stats_kernel, B, 256, 0, s, x, C, mask, area, eps, rs_tmp);
  const int rows = B * HW;
  dim3 grid((rows + 3) / 4);
  const int sp = spatial ? 1 : 0;
  switch (act) {
    case ACT_RELU: launch_k(tip_rms_apply_kernel<ACT_RELU>, grid, 256, 0, s, x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
    case ACT_MISH: launch_k(tip_rms_apply_kernel<ACT_MISH>, grid, 256, 0, s, x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
    case ACT_SILU: launch_k(tip_rms_apply_kernel<ACT_SILU>, grid, 256, 0, s, x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
    default: launch_k(tip_rms_apply_kernel<ACT_ID>, grid, 256, 0, s, x, C, gamma, beta, eps, sp, mask, rs_tmp, out, rows); break;
  }
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Attention: one thread per query, keys and values staged 32 at a time in LDS, online softmax
// ---------------------------------------------------------------------------------------------------------

template <typename T, int D>
__global__ __launch_bounds__(64) void attn_kernel(AttnArgs a) {
  const int qi = blockIdx.x * 64 + threadIdx.x, h = blockIdx.y, n = blockIdx.z, tid = threadIdx.x;
  const int kvh = h / (a.H / a.KV);
  const bool in_range = qi < HW;
  const int qrow = in_range ? qi : 0;
  const T* qkv = (const T*)a.qkv;
  float q[D], acc[D];
  {
    const T* qp = qkv + ((size_t)n * HW + qrow) * a.ldq + a.q_off + h * D;
#pragma unroll
    for (int d = 0; d < D; d++) q[d] = (float)qp[d] * a.scale;
  }
#pragma unroll
  for (int d = 0; d < D; d++) acc[d] = 0.f;
  float m_run = -FLT_MAX, l_run = 0.f;
  __shared__ float ks[32 * D], vs[32 * D], kb[32];
  for (int j0 = 0; j0 < HW; j0 += 32) {
    const int cnt = min(32, HW - j0);
    for (int e = tid; e < 32 * D; e += 64) {
      const int j = e / D, d = e - j * D;
      float kv = 0.f, vv = 0.f;
      if (j < cnt) {
        const T* row = qkv + ((size_t)n * HW + j0 + j) * a.ldq;
        kv = (float)row[a.k_off + kvh * D + d];
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

// Attention on the matrix cores (16-bit handles). A workgroup of twelve waves takes all the queries of one
// (batch row, head), 32 per wave, so each key tile is staged once per head. Keys go in tiles of 64,
// double-buffered in LDS: K ([key][d], RoPE already applied by the projection) and V transposed ([d][key], keys
// permuted as below), each tile loaded into registers one tile ahead of its use. Each wave computes S^T = K Q^T for its 32 queries (keys as rows: a lane holds four
// consecutive keys of one query, so the reductions over keys stay in the lane but for two cross-lane steps), with
// the key mask bias as the accumulator's initial value, then O^T += V^T P^T. P needs no data movement: for a
// 32-key block the B operand of a lane is its own eight probabilities (keys 4g..4g+3 of the block's first 16 and
// of its second 16, g = lane / 16), so V^T holds its keys in that order. The softmax runs online over the 64-key
// tiles (running maximum per query, accumulators rescaled once per tile). Q carries RoPE and the 1/sqrt(d) scale
// and is held in registers as B fragments. The output goes through LDS for 16-byte stores.
constexpr int ATT_QW = 32, ATT_NW = 12, ATT_QB = ATT_QW * ATT_NW, ATT_NQB = (HW + ATT_QB - 1) / ATT_QB;
constexpr int ATT_KT = 64, ATT_NKT = (HW + ATT_KT - 1) / ATT_KT;

// Position of key kk (0..31) of a 32-key block in the permuted V^T rows.
__device__ __forceinline__ int att_kpos(int kk) {
  return kk < 16 ? 8 * (kk >> 2) + (kk & 3) : 8 * ((kk - 16) >> 2) + 4 + ((kk - 16) & 3);
}

// Three workgroups per CU for D <= 32; two for D = 64, whose registers spill at the three-workgroup bound (the
// spill-free kernel is 4 % faster at b10c384h6).
template <typename T, int D>
// The fields that the first loads need lead the arguments (copies of a's) so that they are preloaded into SGPRs
// at wave launch; by-value structs are not.
__global__ __launch_bounds__(ATT_NW * 64, 1) void attn_mfma_kernel(const void* a_qkv, const float* a_mask,
                                                                   int nheads_total, int a_H, int a_KV, int a_ldq,
                                                                   int a_q_off, int a_k_off, int a_v_off, AttnArgs a) {
  static_assert(D == 16 || D == 32 || D == 64, "head dim");
  typedef typename std::conditional<std::is_same<T, f16>::value, half8, bf16x8>::type frag_t;
  constexpr int NT = ATT_NW * 64;
  constexpr int DP = D < 32 ? 32 : D;  // contraction length of S (zero-padded to an MFMA K)
  constexpr int KC = DP / 32, DT = D / 16, QT = ATT_QW / 16, KB = ATT_KT / 32;
  constexpr int HALF = D / 2, NCH = HALF / 8;
  constexpr int KLD = DP + 16, VLD = ATT_KT + 16;  // LDS row strides (160 / 96-byte rows: conflict-free fragments)
  constexpr int KS_SZ = ATT_KT * KLD, VS_SZ = D * VLD;
  constexpr int BUF = (KS_SZ + VS_SZ) * (int)sizeof(T) + ATT_KT * 4;  // bytes per buffer: K, V^T, key bias
  constexpr int OLD = D + 8, OUT = ATT_NW * ATT_QW * OLD * (int)sizeof(T);
  constexpr int NBUF = 2;
  constexpr int LDS = NBUF * BUF > OUT ? NBUF * BUF : OUT;
  constexpr int KU = ATT_KT * NCH, VU = (ATT_KT / 2) * (D / 8);  // staging units: (key, chunk pair), (key pair, chunk)
  static_assert(KU <= NT && VU <= NT && BUF % 16 == 0, "staging layout");
  constexpr float L2E = 1.4426950408889634f;
  __shared__ __align__(16) char smem[LDS];

  const int g0 = blockIdx.x, slot = g0 >> 3, qb = slot % ATT_NQB, nh = (slot / ATT_NQB) * 8 + (g0 & 7);
  if (nh >= nheads_total) return;
  const int h = nh % a_H, n = nh / a_H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int kvh = h / (a_H / a_KV);
  const T* qkv = (const T*)a_qkv;
  const T* kbase = qkv + (size_t)n * HW * a_ldq + a_k_off + kvh * D;
  const T* vbase = qkv + (size_t)n * HW * a_ldq + a_v_off + kvh * D;
  const float* mrow = a_mask + (size_t)n * HW;

  // Zero K's padding columns (head dim 16) in both buffers; staging never writes them.
  if constexpr (DP > D) {
    for (int i = tid; i < NBUF * ATT_KT; i += NT) {
      T* Ks = (T*)(smem + (i / ATT_KT) * BUF) + (i % ATT_KT) * KLD + D;
      *(u32x4*)Ks = u32x4{0, 0, 0, 0};
      *(u32x4*)(Ks + 8) = u32x4{0, 0, 0, 0};
    }
  }

  // Q fragments: query qbase + qt*16 + l16, dims kc*32 + 8g .. +8 (zero beyond the head dim and the board).
  const int qbase = qb * ATT_QB + wave * ATT_QW;
  frag_t qf[QT][KC];
#pragma unroll
  for (int qt = 0; qt < QT; qt++) {
    const int qi = qbase + qt * 16 + l16;
#pragma unroll
    for (int kc = 0; kc < KC; kc++) {
      const int d0 = kc * 32 + 8 * g;
      frag_t r;
#pragma unroll
      for (int e = 0; e < 8; e++) r[e] = to_t<T>(0.f);
      if (qi < HW && d0 < D) {
        const T* qp = qkv + ((size_t)n * HW + qi) * a_ldq + a_q_off + h * D;
        const frag_t x = *(const frag_t*)(qp + d0);
#pragma unroll
        for (int e = 0; e < 8; e++) r[e] = to_t<T>((float)x[e] * a.scale);
      }
      qf[qt][kc] = r;
    }
  }

  // Staging of one key tile: registers (fetch) then LDS (stash).
  const int ku_key = tid / NCH, ku_c = (tid % NCH) * 8;            // K unit: key, first dim of the low chunk
  const int vu_pair = tid / (D / 8), vu_c = (tid % (D / 8)) * 8;  // V unit: key pair, first dim of the chunk
  struct Stage {
    frag_t kx0, kx1, vx0, vx1;
    float mk = 0.f;
  };
  // Keys past the board read the last key's rows (finite values): their bias of -1e30 gives them probability 0.
  auto fetch = [&](int t, Stage& st) {
    const int k0 = t * ATT_KT;
    if (tid < KU) {
      const int key = min(k0 + ku_key, HW - 1);
      const T* kp = kbase + (size_t)key * a_ldq + ku_c;
      st.kx0 = *(const frag_t*)kp;
      st.kx1 = *(const frag_t*)(kp + HALF);
    }
    if (tid < VU) {
      const int key = min(k0 + 2 * vu_pair, HW - 1), key1 = min(k0 + 2 * vu_pair + 1, HW - 1);
      st.vx0 = *(const frag_t*)(vbase + (size_t)key * a_ldq + vu_c);
      st.vx1 = *(const frag_t*)(vbase + (size_t)key1 * a_ldq + vu_c);
    }
    if (tid < ATT_KT) {
      const int key = k0 + tid;
      st.mk = key < HW ? mrow[key] * 3e4f - 3e4f : -1e30f;
    }
  };
  auto stash = [&](int b, const Stage& st) {
    T* Ks = (T*)(smem + b * BUF);
    T* Vs = Ks + KS_SZ;
    float* kbias = (float*)(Vs + VS_SZ);
    if (tid < KU) {
      *(frag_t*)(Ks + ku_key * KLD + ku_c) = st.kx0;
      *(frag_t*)(Ks + ku_key * KLD + ku_c + HALF) = st.kx1;
    }
    if (tid < VU) {
      const int kk = 2 * vu_pair, pos = (kk & ~31) + att_kpos(kk & 31);
      const u32x4 w0 = __builtin_bit_cast(u32x4, st.vx0), w1 = __builtin_bit_cast(u32x4, st.vx1);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        // Element e of both keys: the 16-bit halves of word e / 2.
        const unsigned a0 = w0[e >> 1], a1 = w1[e >> 1];
        *(unsigned*)(Vs + (vu_c + e) * VLD + pos) =
            (e & 1) ? (a0 >> 16) | (a1 & 0xffff0000u) : (a0 & 0xffffu) | (a1 << 16);
      }
    }
    if (tid < ATT_KT) kbias[tid] = st.mk;
  };

  // O^T tiles, and in tile DT every query's sum of its 16-bit numerators (an all-ones A operand: the MFMA pipe,
  // which this kernel leaves idle most of the time, adds them instead of the VALU).
  floatx4 o[DT + 1][QT];
  float mref[QT];
#pragma unroll
  for (int qt = 0; qt < QT; qt++) {
    mref[qt] = -FLT_MAX;
#pragma unroll
    for (int dt = 0; dt <= DT; dt++) o[dt][qt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Max over the four lane groups that hold one query's keys: lanes j and j ^ 16, then j and j ^ 32, through the
  // gfx950 lane-swap instructions (no LDS round trip). v_permlane16_swap exchanges the odd rows of 16 lanes of its
  // first operand with the even rows of its second, so with both holding v each lane ends with {v[j], v[j ^ 16]};
  // v_permlane32_swap does the same for halves ({v[j], v[j ^ 32]}). Written as inline assembly: the compiler's
  // builtins for these instructions fold the two results into one when both operands hold the same value. The
  // s_nop covers the VALU-write to permlane-read hazard on the operands.
  auto xmax = [](float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    float c = fmaxf(a, b), d = c;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
    return fmaxf(c, d);
  };
  // S^T tiles [key tile][query tile] of one 64-key tile, the key bias as initial accumulator.
  auto scores = [&](int b, floatx4 (&sc)[2 * KB][QT]) {
    const T* Ks = (const T*)(smem + b * BUF);
    const float* kbias = (const float*)(Ks + KS_SZ + VS_SZ);
#pragma unroll
    for (int kt = 0; kt < 2 * KB; kt++) {
      frag_t kf[KC];
#pragma unroll
      for (int kc = 0; kc < KC; kc++) kf[kc] = *(const frag_t*)(Ks + (kt * 16 + l16) * KLD + kc * 32 + 8 * g);
      const floatx4 bias = *(const floatx4*)(kbias + kt * 16 + 4 * g);
#pragma unroll
      for (int qt = 0; qt < QT; qt++) {
        floatx4 c = bias;
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
          if constexpr (std::is_same<T, f16>::value)
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kc], qf[qt][kc], c, 0, 0, 0);
          else
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kc], qf[qt][kc], c, 0, 0, 0);
        }
        sc[kt][qt] = c;
      }
    }
  };
  // Numerators as B fragments of the two 32-key blocks, relative to a reference maximum per query that moves
  // lazily: only when some query of the wave would see a numerator above 2^8 (its tile maximum more than eight
  // binary orders above the reference) are the reference maxima raised to the running maxima, and the
  // accumulators (the sums' tile with them) rescaled, in one wave-uniform branch. Otherwise every numerator stays below 2^8 (in
  // range and at full relative precision as a 16-bit operand), and O, the sums and the numerators all stay
  // relative to the same unchanged reference.
  auto softmax = [&](const floatx4 (&sc)[2 * KB][QT], frag_t (&pf)[KB][QT]) {
    float mx[QT];
    bool grow = false;
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
      float m = sc[0][qt][0];
#pragma unroll
      for (int kt = 0; kt < 2 * KB; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) m = fmaxf(m, sc[kt][qt][r]);
      mx[qt] = xmax(m);
      grow |= (mx[qt] - mref[qt]) * L2E > 8.f;
    }
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int qt = 0; qt < QT; qt++) {
        const float mnew = fmaxf(mref[qt], mx[qt]);
        const float alpha = __builtin_amdgcn_exp2f((mref[qt] - mnew) * L2E);
#pragma unroll
        for (int dt = 0; dt <= DT; dt++) o[dt][qt] *= alpha;
        mref[qt] = mnew;
      }
    }
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
      const float ml = mref[qt] * L2E;
#pragma unroll
      for (int kb = 0; kb < KB; kb++) {
        frag_t pr;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
          for (int r = 0; r < 4; r++) pr[4 * j + r] = to_t<T>(__builtin_amdgcn_exp2f(fmaf(sc[2 * kb + j][qt][r], L2E, -ml)));
        pf[kb][qt] = pr;
      }
    }
  };
  // O^T += V^T P^T.
  auto pv = [&](int b, const frag_t (&pf)[KB][QT]) {
    const T* Vs = (const T*)(smem + b * BUF) + KS_SZ;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
#pragma unroll
      for (int kb = 0; kb < KB; kb++) {
        const frag_t vf = *(const frag_t*)(Vs + (dt * 16 + l16) * VLD + kb * 32 + 8 * g);
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
          if constexpr (std::is_same<T, f16>::value)
            o[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[kb][qt], o[dt][qt], 0, 0, 0);
          else
            o[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[kb][qt], o[dt][qt], 0, 0, 0);
        }
      }
    }
    frag_t ones;
#pragma unroll
    for (int e = 0; e < 8; e++) ones[e] = to_t<T>(1.f);
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
      for (int qt = 0; qt < QT; qt++) {
        if constexpr (std::is_same<T, f16>::value)
          o[DT][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[kb][qt], o[DT][qt], 0, 0, 0);
        else
          o[DT][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[kb][qt], o[DT][qt], 0, 0, 0);
      }
  };

  // Per tile t: the loads of tile t + 1 in flight during tile t's scores, softmax and O update; then tile t + 1
  // into the other buffer and one barrier.
  Stage st;
  fetch(0, st);
  stash(0, st);
  __syncthreads();
  for (int t = 0; t < ATT_NKT; t++) {
    if (t + 1 < ATT_NKT) fetch(t + 1, st);
    floatx4 sc[2 * KB][QT];
    scores(t & 1, sc);
    frag_t pf[KB][QT];
    softmax(sc, pf);
    pv(t & 1, pf);
    if (t + 1 < ATT_NKT) stash((t + 1) & 1, st);
    __syncthreads();
  }

  // Normalize by the sums' tile (every element of a query's column holds its sum), transpose through LDS
  // ([wave][query][d]) and store 16-byte vectors of the queries on the board.
  T* Os = (T*)smem + wave * ATT_QW * OLD;
#pragma unroll
  for (int qt = 0; qt < QT; qt++) {
    const float l = o[DT][qt][0];
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int r = 0; r < 4; r++) Os[(qt * 16 + l16) * OLD + dt * 16 + 4 * g + r] = to_t<T>(o[dt][qt][r] * inv);
  }
  __syncthreads();
  for (int e = lane; e < ATT_QW * (D / 8); e += 64) {
    const int qq = e / (D / 8), d0 = (e % (D / 8)) * 8, qi = qbase + qq;
    if (qi < HW) *(u32x4*)((T*)a.out + ((size_t)n * HW + qi) * a.ldo + h * D + d0) = *(const u32x4*)(Os + qq * OLD + d0);
  }
}

template <typename T, int D>
static void attn_mfma_d(const AttnArgs& a, int B, hipStream_t s) {
  const int nh = B * a.H;
  dim3 grid((nh + 7) / 8 * 8 * ATT_NQB);
  launch_k(attn_mfma_kernel<T, D>, grid, ATT_NW * 64, 0, s, a.qkv, a.mask, nh, a.H, a.KV, a.ldq, a.q_off, a.k_off,
           a.v_off, a);
}

template <typename T, int D>
static void attn_d(const AttnArgs& a, int B, hipStream_t s) {
  dim3 grid((HW + 63) / 64, a.H, B);
  launch_k(attn_kernel<T, D>, grid, 64, 0, s, a);
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

template <typename T>
static void attn_mfma_t(const AttnArgs& a, int B, hipStream_t s) {
  if (a.dq != a.dv) throw std::runtime_error("attention: dq != dv unsupported");
  // 16-byte rows of q/k/v and of the output.
  if (a.ldq % 8 || a.q_off % 8 || a.k_off % 8 || a.v_off % 8 || a.ldo % 8)
    throw std::runtime_error("attention: q/k/v and output offsets must be multiples of 8 elements");
  switch (a.dq) {
    case 16: attn_mfma_d<T, 16>(a, B, s); break;
    case 32: attn_mfma_d<T, 32>(a, B, s); break;
    case 64: attn_mfma_d<T, 64>(a, B, s); break;
    default: throw std::runtime_error("attention: head dim must be 16, 32 or 64");
  }
}

void launch_attention(int prec, const AttnArgs& a, int B, hipStream_t s) {
  if (prec == PREC_F16) attn_mfma_t<f16>(a, B, s);
  else if (prec == PREC_BF16) attn_mfma_t<bf16>(a, B, s);
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
  else v = sizeof(T) == 2 ? act16<ACT_MISH>(a, 1.f) : act_f<ACT_MISH>(a);  // as the fused FFN epilogue
  h[r * ldh + f] = to_t<T>(v);
}

void launch_ffn_act(int prec, const float* u, int ldu, int F, bool gated, void* h, int ldh, int rows, hipStream_t s) {
  const size_t total = (size_t)rows * F;
  dim3 grid((unsigned)((total + 255) / 256));
#define KGX_FFN(T) \
  if (gated) launch_k(ffn_act_kernel<T, true>, grid, 256, 0, s, u, ldu, F, (T*)h, ldh, rows); \
  else launch_k(ffn_act_kernel<T, false>, grid, 256, 0, s, u, ldu, F, (T*)h, ldh, rows);
  if (prec == PREC_F16) { KGX_FFN(f16) }
  else if (prec == PREC_BF16) { KGX_FFN(bf16) }
  else { KGX_FFN(float) }
#undef KGX_FFN
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
