// HIP kernels for gfx950 (CDNA4): the KataGo forward pass on an NHWC activation layout ([batch * 361][C],
// channels contiguous), which is also the token layout of the transformer blocks.
//
// Winograd F(4x4,3x3) follows crates/katago-nn-burn/src/wino/kernels.rs (input transform :79-179, output
// transform :312-384, filter transform :36-69); the GEMMs run on MFMA (v_mfma_f32_16x16x32_{f16,bf16},
// v_mfma_f32_16x16x4_f32) with float accumulation. Pooling follows tools/bin2onnx/bin2onnx.py:1203-1247,
// RMSNorm tools/bin2onnx/bin2onnx.py:1338-1348 and crates/katago-nn-burn/src/tfk/kernels.rs:275-305, attention
// crates/katago-nn-burn/src/tfk/kernels.rs:442-613.
#include "kgx_kernels.h"

#include <cfloat>
#include <type_traits>
#include <cmath>
#include <stdexcept>
#include <string>

namespace kgx {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define KGX_CHECK_LAUNCH()                                                              \
  do {                                                                                  \
    hipError_t e_ = hipGetLastError();                                                  \
    if (e_ != hipSuccess) throw std::runtime_error(std::string("kernel launch: ") + hipGetErrorString(e_)); \
  } while (0)

// ---------------------------------------------------------------------------------------------------------
// Element helpers
// ---------------------------------------------------------------------------------------------------------

template <int ACT>
__device__ __forceinline__ float act_f(float a) {
  if constexpr (ACT == ACT_RELU) {
    return fmaxf(a, 0.f);
  } else if constexpr (ACT == ACT_MISH) {
    // a * tanh(softplus(a)); with e = exp(a), tanh(log(1 + e)) = e (e + 2) / (e (e + 2) + 2). Softplus is the
    // identity above 20 (burn's threshold), where tanh is 1 in float.
    if (a > 20.f) return a;
    const float e = __expf(a);
    const float n = e * (e + 2.f);
    return a * n * __builtin_amdgcn_rcpf(n + 2.f);
  } else if constexpr (ACT == ACT_SILU) {
    return a * __builtin_amdgcn_rcpf(__expf(-a) + 1.f);  // x / (exp(-x) + 1)
  } else {
    return a;
  }
}

template <typename T>
__device__ __forceinline__ T to_t(float v) { return (T)v; }

template <typename T> struct Tile;
template <> struct Tile<float> { static constexpr int BK = 16, VEC = 4; };
template <> struct Tile<f16> { static constexpr int BK = 32, VEC = 8; };
template <> struct Tile<bf16> { static constexpr int BK = 32, VEC = 8; };

// ---------------------------------------------------------------------------------------------------------
// Winograd input transform (with the BN + activation + mask prologue)
// ---------------------------------------------------------------------------------------------------------

// B^T d over 6 values (rows 4,0,-5,0,1,0 / 0,-4,-4,1,1,0 / 0,4,-4,-1,1,0 / 0,-2,-1,2,1,0 / 0,2,-1,-2,1,0 /
// 0,4,0,-5,0,1).
__device__ __forceinline__ void bt6(float z0, float z1, float z2, float z3, float z4, float z5, float* o) {
  o[0] = 4.f * z0 - 5.f * z2 + z4;
  o[1] = -4.f * z1 - 4.f * z2 + z3 + z4;
  o[2] = 4.f * z1 - 4.f * z2 - z3 + z4;
  o[3] = -2.f * z1 - z2 + 2.f * z3 + z4;
  o[4] = 2.f * z1 - z2 - 2.f * z3 + z4;
  o[5] = 4.f * z1 - 5.f * z3 + z5;
}

// A^T m over 6 values (rows 1,1,1,1,1,0 / 0,1,-1,2,-2,0 / 0,1,1,4,4,0 / 0,1,-1,8,-8,1).
__device__ __forceinline__ void at6(float z0, float z1, float z2, float z3, float z4, float z5, float* o) {
  o[0] = z0 + z1 + z2 + z3 + z4;
  o[1] = (z1 - z2) + 2.f * (z3 - z4);
  o[2] = (z1 + z2) + 4.f * (z3 + z4);
  o[3] = (z1 - z2) + 8.f * (z3 - z4) + z5;
}

// One thread per (tile, channel), channels along x: reads of a board point are coalesced over channels
// (NHWC), writes V[p][t][c] too. Tile t = (n * 5 + tile_y) * 5 + tile_x; its 6x6 window starts at
// (4 tile_y - 1, 4 tile_x - 1), zero outside the board.
template <typename T, bool PRO, int ACT, bool NCHW>
__global__ __launch_bounds__(256) void wino_in_kernel(const float* __restrict__ x, int ldx, Prologue pro,
                                                      T* __restrict__ V, int B, int C, int c_pad, int t_pad) {
  const int c = blockIdx.x * 64 + threadIdx.x;
  const int t = blockIdx.y * 4 + threadIdx.y;
  if (c >= c_pad || t >= t_pad) return;
  float d[36];
  if (t < B * TILES && c < C) {
    const int n = t / TILES, tile = t - n * TILES;
    const int ty = tile / TILES_X, tx = tile - ty * TILES_X;
    float sc = 0.f, bi = 0.f, pb = 0.f;
    if constexpr (PRO) {
      sc = pro.scale[c];
      bi = pro.bias[c];
      if (pro.prebias) pb = pro.prebias[(size_t)n * pro.ld_prebias + c];
    }
#pragma unroll
    for (int sy = 0; sy < 6; sy++) {
#pragma unroll
      for (int sx = 0; sx < 6; sx++) {
        const int yy = ty * 4 + sy - 1, xx = tx * 4 + sx - 1;
        float v = 0.f;
        if (yy >= 0 && yy < POS && xx >= 0 && xx < POS) {
          const int pos = yy * POS + xx;
          if constexpr (NCHW) v = x[((size_t)n * C + c) * HW + pos];
          else v = x[((size_t)n * HW + pos) * ldx + c];
          if constexpr (PRO) v = act_f<ACT>((v + pb) * sc + bi) * pro.mask[(size_t)n * HW + pos];
        }
        d[sy * 6 + sx] = v;
      }
    }
    float r[36];
#pragma unroll
    for (int sy = 0; sy < 6; sy++)
      bt6(d[sy * 6], d[sy * 6 + 1], d[sy * 6 + 2], d[sy * 6 + 3], d[sy * 6 + 4], d[sy * 6 + 5], &r[sy * 6]);
#pragma unroll
    for (int sx = 0; sx < 6; sx++) {
      float o[6];
      bt6(r[sx], r[6 + sx], r[12 + sx], r[18 + sx], r[24 + sx], r[30 + sx], o);
#pragma unroll
      for (int k = 0; k < 6; k++) d[k * 6 + sx] = o[k];
    }
  } else {
#pragma unroll
    for (int p = 0; p < 36; p++) d[p] = 0.f;
  }
#pragma unroll
  for (int p = 0; p < 36; p++) V[((size_t)p * t_pad + t) * c_pad + c] = to_t<T>(d[p]);
}

template <typename T, bool PRO, bool NCHW>
static void wino_in_act(int act, dim3 grid, dim3 block, hipStream_t s, const float* x, int ldx, const Prologue& pro,
                        T* V, int B, int C, int c_pad, int t_pad) {
  switch (act) {
    case ACT_RELU: wino_in_kernel<T, PRO, ACT_RELU, NCHW><<<grid, block, 0, s>>>(x, ldx, pro, V, B, C, c_pad, t_pad); break;
    case ACT_MISH: wino_in_kernel<T, PRO, ACT_MISH, NCHW><<<grid, block, 0, s>>>(x, ldx, pro, V, B, C, c_pad, t_pad); break;
    case ACT_SILU: wino_in_kernel<T, PRO, ACT_SILU, NCHW><<<grid, block, 0, s>>>(x, ldx, pro, V, B, C, c_pad, t_pad); break;
    default: wino_in_kernel<T, PRO, ACT_ID, NCHW><<<grid, block, 0, s>>>(x, ldx, pro, V, B, C, c_pad, t_pad); break;
  }
}

template <typename T>
static void wino_in_t(const float* x, int ldx, bool nchw, const Prologue& pro, T* V, int B, int C, int c_pad,
                      int t_pad, hipStream_t s) {
  dim3 block(64, 4), grid((c_pad + 63) / 64, t_pad / 4);
  const bool p = pro.scale != nullptr;
  if (nchw) {
    if (p) throw std::runtime_error("wino_in: prologue on NCHW input");
    wino_in_act<T, false, true>(ACT_ID, grid, block, s, x, ldx, pro, V, B, C, c_pad, t_pad);
  } else if (p) {
    wino_in_act<T, true, false>(pro.act, grid, block, s, x, ldx, pro, V, B, C, c_pad, t_pad);
  } else {
    wino_in_act<T, false, false>(ACT_ID, grid, block, s, x, ldx, pro, V, B, C, c_pad, t_pad);
  }
}

void launch_wino_in(int prec, const float* x, int ldx, bool nchw, const Prologue& pro, void* V, int B, int C,
                    int c_pad, int t_pad, hipStream_t s) {
  if (t_pad % 4 != 0 || t_pad < B * TILES || c_pad < C) throw std::runtime_error("wino_in: bad padding");
  if (prec == PREC_F16) wino_in_t<f16>(x, ldx, nchw, pro, (f16*)V, B, C, c_pad, t_pad, s);
  else if (prec == PREC_BF16) wino_in_t<bf16>(x, ldx, nchw, pro, (bf16*)V, B, C, c_pad, t_pad, s);
  else wino_in_t<float>(x, ldx, nchw, pro, (float*)V, B, C, c_pad, t_pad, s);
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Winograd output transform (+ per-(row, channel) bias, + residual accumulate)
// ---------------------------------------------------------------------------------------------------------

template <bool ACC, bool BIAS>
__global__ __launch_bounds__(256) void wino_out_kernel(const float* __restrict__ M, int oc_pad, int t_pad,
                                                       float* __restrict__ out, int ldo, int OC,
                                                       const float* __restrict__ colbias, int ldcb, int B) {
  const int oc = blockIdx.x * 64 + threadIdx.x;
  const int t = blockIdx.y * 4 + threadIdx.y;
  if (oc >= OC || t >= B * TILES) return;
  float m[36];
#pragma unroll
  for (int p = 0; p < 36; p++) m[p] = M[((size_t)p * t_pad + t) * oc_pad + oc];
  float r[24];  // [6 rows][4]
#pragma unroll
  for (int sy = 0; sy < 6; sy++) at6(m[sy * 6], m[sy * 6 + 1], m[sy * 6 + 2], m[sy * 6 + 3], m[sy * 6 + 4], m[sy * 6 + 5], &r[sy * 4]);
  float o[16];
#pragma unroll
  for (int sx = 0; sx < 4; sx++) {
    float c4[4];
    at6(r[sx], r[4 + sx], r[8 + sx], r[12 + sx], r[16 + sx], r[20 + sx], c4);
#pragma unroll
    for (int k = 0; k < 4; k++) o[k * 4 + sx] = c4[k];
  }
  const int n = t / TILES, tile = t - n * TILES;
  const int ty = tile / TILES_X, tx = tile - ty * TILES_X;
  const float bias = BIAS ? colbias[(size_t)n * ldcb + oc] : 0.f;
#pragma unroll
  for (int sy = 0; sy < 4; sy++)
#pragma unroll
    for (int sx = 0; sx < 4; sx++) {
      const int yy = ty * 4 + sy, xx = tx * 4 + sx;
      if (yy < POS && xx < POS) {
        const size_t idx = ((size_t)n * HW + yy * POS + xx) * ldo + oc;
        const float v = o[sy * 4 + sx] + bias;
        if (ACC) out[idx] += v;
        else out[idx] = v;
      }
    }
}

void launch_wino_out(const float* M, int oc_pad, int t_pad, float* out, int ldo, int OC, const float* colbias,
                     int ld_colbias, bool accumulate, int B, hipStream_t s) {
  dim3 block(64, 4), grid((OC + 63) / 64, (B * TILES + 3) / 4);
  if (accumulate) {
    if (colbias) wino_out_kernel<true, true><<<grid, block, 0, s>>>(M, oc_pad, t_pad, out, ldo, OC, colbias, ld_colbias, B);
    else wino_out_kernel<true, false><<<grid, block, 0, s>>>(M, oc_pad, t_pad, out, ldo, OC, colbias, ld_colbias, B);
  } else {
    if (colbias) wino_out_kernel<false, true><<<grid, block, 0, s>>>(M, oc_pad, t_pad, out, ldo, OC, colbias, ld_colbias, B);
    else wino_out_kernel<false, false><<<grid, block, 0, s>>>(M, oc_pad, t_pad, out, ldo, OC, colbias, ld_colbias, B);
  }
  KGX_CHECK_LAUNCH();
}

// Filter transform in double, rounded once to float: U[p][o][i] = (G g G^T)[p] with G's rows
// (1/4, 0, 0), (-1/6, -1/6, -1/6), (-1/6, 1/6, -1/6), (1/24, 1/12, 1/6), (1/24, -1/12, 1/6), (0, 0, 1)
// (wino/kernels.rs:39-48). Padding is zero.
void wino_filter_host(const float* w, int oc, int ic, int oc_pad, int ic_pad, float* U) {
  auto g6 = [](const double z[3], double o[6]) {
    o[0] = 0.25 * z[0];
    o[1] = (-z[0] - z[1] - z[2]) / 6.0;
    o[2] = (-z[0] + z[1] - z[2]) / 6.0;
    o[3] = (z[0] + 2.0 * z[1] + 4.0 * z[2]) / 24.0;
    o[4] = (z[0] - 2.0 * z[1] + 4.0 * z[2]) / 24.0;
    o[5] = z[2];
  };
  for (size_t k = 0; k < (size_t)36 * oc_pad * ic_pad; k++) U[k] = 0.f;
  for (int o = 0; o < oc; o++)
    for (int i = 0; i < ic; i++) {
      double g[9];
      for (int k = 0; k < 9; k++) g[k] = w[((size_t)o * ic + i) * 9 + k];
      double rows[3][6];
      for (int y = 0; y < 3; y++) g6(&g[3 * y], rows[y]);
      for (int xx = 0; xx < 6; xx++) {
        double col[3] = {rows[0][xx], rows[1][xx], rows[2][xx]}, t6[6];
        g6(col, t6);
        for (int y = 0; y < 6; y++) U[(((size_t)(y * 6 + xx)) * oc_pad + o) * ic_pad + i] = (float)t6[y];
      }
    }
}

// ---------------------------------------------------------------------------------------------------------
// MFMA GEMM: C[z][m][n] = sum_k A[z][m][k] * Bt[z][n][k]
// ---------------------------------------------------------------------------------------------------------
// 64x64 output tile per 256-thread workgroup, 4 waves in 2x2, each wave 32x32 = 2x2 MFMA 16x16 blocks.
// A and B tiles of BK (32 for 16-bit types, 16 for float) are staged in LDS with a 16-byte row pad; the next
// tile is prefetched into registers while the current one feeds the MFMAs. A may be float activations, in
// which case the BN + activation + mask prologue runs on load and the values are converted to T.

enum { E_RES = 1, E_BIAS = 2, E_MASK = 4, E_OUT_T = 8 };

template <typename T, bool AF, bool PRO, int ACT, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  constexpr int BM = 64, BN = 64;
  constexpr int BK = Tile<T>::BK, VEC = Tile<T>::VEC;
  constexpr int LDK = BK + VEC;
  constexpr int KV = BK / VEC;  // 16-byte vectors per tile row (4)
  __shared__ __align__(16) T As[BM * LDK];
  __shared__ __align__(16) T Bs[BN * LDK];
  typedef uint4 vec_t;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int z = blockIdx.z;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int lrow = tid / KV, lk = (tid % KV) * VEC;
  const int M = g.M, N = g.N, K = g.K;

  const T* At = (const T*)g.A + (size_t)z * g.sA;
  const float* Af = (const float*)g.A + (size_t)z * g.sA;
  const T* Bt = (const T*)g.Bt + (size_t)z * g.sB;

  vec_t ra, rb;
  auto load_a = [&](int k0) {
    const int m = m0 + lrow, k = k0 + lk;
    if constexpr (!AF) {
      if (m < M && k < K) ra = *(const vec_t*)(At + (size_t)m * g.lda + k);
      else ra = vec_t{0, 0, 0, 0};
    } else {
      T v[VEC];
      if (m < M && k < K) {
        float f[VEC];
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
          const float4 q = *(const float4*)(Af + (size_t)m * g.lda + k + e);
          f[e] = q.x; f[e + 1] = q.y; f[e + 2] = q.z; f[e + 3] = q.w;
        }
        if constexpr (PRO) {
          const float mk = g.pro.mask[m];
          const float* pb = g.pro.prebias ? g.pro.prebias + (size_t)(m / HW) * g.pro.ld_prebias : nullptr;
#pragma unroll
          for (int e = 0; e < VEC; e++) {
            float a = f[e];
            if (pb) a += pb[k + e];
            f[e] = act_f<ACT>(a * g.pro.scale[k + e] + g.pro.bias[k + e]) * mk;
          }
        }
#pragma unroll
        for (int e = 0; e < VEC; e++) v[e] = to_t<T>(f[e]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; e++) v[e] = to_t<T>(0.f);
      }
      ra = *(const vec_t*)v;
    }
  };
  auto load_b = [&](int k0) {
    const int nn = n0 + lrow, k = k0 + lk;
    if (nn < N && k < K) rb = *(const vec_t*)(Bt + (size_t)nn * g.ldb + k);
    else rb = vec_t{0, 0, 0, 0};
  };

  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  load_b(0);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    *(vec_t*)(&As[lrow * LDK + lk]) = ra;
    *(vec_t*)(&Bs[lrow * LDK + lk]) = rb;
    __syncthreads();
    if (k0 + BK < K) {
      load_a(k0 + BK);
      load_b(k0 + BK);
    }
    const int r16 = lane & 15, g4 = lane >> 4;
    if constexpr (sizeof(T) == 2) {
      typedef typename std::conditional<std::is_same<T, f16>::value, half8, bf16x8>::type frag_t;
      frag_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = *(const frag_t*)(&As[(wm * 32 + i * 16 + r16) * LDK + g4 * 8]);
#pragma unroll
      for (int j = 0; j < 2; j++) b[j] = *(const frag_t*)(&Bs[(wn * 32 + j * 16 + r16) * LDK + g4 * 8]);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          if constexpr (std::is_same<T, f16>::value)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    } else {
#pragma unroll
      for (int kk = 0; kk < BK; kk += 4) {
        float a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = As[(wm * 32 + i * 16 + r16) * LDK + kk + g4];
#pragma unroll
        for (int j = 0; j < 2; j++) b[j] = Bs[(wn * 32 + j * 16 + r16) * LDK + kk + g4];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
          for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // Output element (i, j, r) of this lane: row wm*32 + i*16 + 4*(lane/16) + r, column wn*32 + j*16 + lane%16.
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
        const int nn = n0 + wn * 32 + j * 16 + (lane & 15);
        if (m < M && nn < N) {
          float v = acc[i][j][r];
          if constexpr (EPI & E_BIAS) v += g.colbias[(size_t)(m / HW) * g.ld_colbias + nn];
          if constexpr (EPI & E_MASK) v *= g.rowmask[m];
          if constexpr (EPI & E_RES) v += g.residual[(size_t)m * g.ldr + nn];
          if constexpr (EPI & E_OUT_T) ((T*)g.C)[(size_t)z * g.sC + (size_t)m * g.ldc + nn] = to_t<T>(v);
          else ((float*)g.C)[(size_t)z * g.sC + (size_t)m * g.ldc + nn] = v;
        }
      }
}

template <typename T, bool AF, bool PRO, int ACT>
static void gemm_epi(const GemmArgs& g, dim3 grid, hipStream_t s) {
  int epi = (g.residual ? E_RES : 0) | (g.colbias ? E_BIAS : 0) | (g.rowmask ? E_MASK : 0) | (g.out_t ? E_OUT_T : 0);
  switch (epi) {
    case 0: gemm_kernel<T, AF, PRO, ACT, 0><<<grid, 256, 0, s>>>(g); break;
    case E_RES: gemm_kernel<T, AF, PRO, ACT, E_RES><<<grid, 256, 0, s>>>(g); break;
    case E_MASK | E_RES: gemm_kernel<T, AF, PRO, ACT, E_MASK | E_RES><<<grid, 256, 0, s>>>(g); break;
    case E_OUT_T: gemm_kernel<T, AF, PRO, ACT, E_OUT_T><<<grid, 256, 0, s>>>(g); break;
    default: throw std::runtime_error("gemm: unsupported epilogue combination " + std::to_string(epi));
  }
}

template <typename T>
static void gemm_t(const GemmArgs& g, hipStream_t s) {
  dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, g.Z);
  if (!g.a_float) {
    gemm_epi<T, false, false, ACT_ID>(g, grid, s);
  } else if (!g.pro.scale) {
    gemm_epi<T, true, false, ACT_ID>(g, grid, s);
  } else {
    switch (g.pro.act) {
      case ACT_RELU: gemm_epi<T, true, true, ACT_RELU>(g, grid, s); break;
      case ACT_MISH: gemm_epi<T, true, true, ACT_MISH>(g, grid, s); break;
      case ACT_SILU: gemm_epi<T, true, true, ACT_SILU>(g, grid, s); break;
      default: gemm_epi<T, true, true, ACT_ID>(g, grid, s); break;
    }
  }
}

void launch_gemm(int prec, const GemmArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0) return;
  const int vec = prec == PREC_F32 ? 4 : 8;
  if (g.K % vec != 0 || g.lda % vec != 0 || g.ldb % vec != 0) throw std::runtime_error("gemm: K and strides must be multiples of the vector width");
  if (prec == PREC_F16) gemm_t<f16>(g, s);
  else if (prec == PREC_BF16) gemm_t<bf16>(g, s);
  else gemm_t<float>(g, s);
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Direct odd-k convolution (float): one thread per (oc, point, row)
// ---------------------------------------------------------------------------------------------------------

template <bool PRO, int ACT, bool NCHW>
__global__ __launch_bounds__(64) void conv_direct_kernel(const float* __restrict__ x, int ldx, Prologue pro, int IC,
                                                         const float* __restrict__ w, int OC, int ky, int kx, int dy,
                                                         int dx, float* __restrict__ out, int ldo,
                                                         const float* __restrict__ colbias, int ldcb, int accumulate) {
  const int oc = blockIdx.x * 64 + threadIdx.x;
  const int pos = blockIdx.y, n = blockIdx.z;
  if (oc >= OC) return;
  const int py = pos / POS, px = pos - py * POS;
  const int oy = (ky / 2) * dy, ox = (kx / 2) * dx;
  float acc = 0.f;
  for (int i = 0; i < IC; i++) {
    float sc = 0.f, bi = 0.f, pb = 0.f;
    if constexpr (PRO) {
      sc = pro.scale[i];
      bi = pro.bias[i];
      if (pro.prebias) pb = pro.prebias[(size_t)n * pro.ld_prebias + i];
    }
    for (int a = 0; a < ky; a++) {
      const int sy = py + a * dy - oy;
      if (sy < 0 || sy >= POS) continue;
      for (int b = 0; b < kx; b++) {
        const int sx = px + b * dx - ox;
        if (sx < 0 || sx >= POS) continue;
        const int sp = sy * POS + sx;
        float v = NCHW ? x[((size_t)n * IC + i) * HW + sp] : x[((size_t)n * HW + sp) * ldx + i];
        if constexpr (PRO) v = act_f<ACT>((v + pb) * sc + bi) * pro.mask[(size_t)n * HW + sp];
        acc += v * w[(((size_t)i * ky + a) * kx + b) * OC + oc];
      }
    }
  }
  if (colbias) acc += colbias[(size_t)n * ldcb + oc];
  float* o = out + ((size_t)n * HW + pos) * ldo + oc;
  *o = accumulate ? *o + acc : acc;
}

void launch_conv_direct(const float* x, int ldx, bool nchw, const Prologue& pro, int IC, const float* w, int OC,
                        int ky, int kx, int dy, int dx, float* out, int ldo, const float* colbias, int ld_colbias,
                        bool accumulate, int B, hipStream_t s) {
  dim3 grid((OC + 63) / 64, HW, B);
  const bool p = pro.scale != nullptr;
#define KGX_CD(P, A, N) conv_direct_kernel<P, A, N><<<grid, 64, 0, s>>>(x, ldx, pro, IC, w, OC, ky, kx, dy, dx, out, ldo, colbias, ld_colbias, accumulate ? 1 : 0)
  if (nchw) {
    if (p) throw std::runtime_error("conv_direct: prologue on NCHW input");
    KGX_CD(false, ACT_ID, true);
  } else if (!p) {
    KGX_CD(false, ACT_ID, false);
  } else {
    switch (pro.act) {
      case ACT_RELU: KGX_CD(true, ACT_RELU, false); break;
      case ACT_MISH: KGX_CD(true, ACT_MISH, false); break;
      case ACT_SILU: KGX_CD(true, ACT_SILU, false); break;
      default: KGX_CD(true, ACT_ID, false); break;
    }
  }
#undef KGX_CD
  KGX_CHECK_LAUNCH();
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
  mask_prep_kernel<<<B, 256, 0, s>>>(bin, nin, mask, area, s1, s2);
  KGX_CHECK_LAUNCH();
}

template <bool VALUE, bool PRO, int ACT>
__global__ __launch_bounds__(256) void pool_kernel(const float* __restrict__ x, int ldx, int coff, int C, Prologue pro,
                                                   const float* __restrict__ area, const float* __restrict__ s1,
                                                   const float* __restrict__ s2, float* __restrict__ out) {
  const int c = blockIdx.x * 64 + threadIdx.x, b = blockIdx.y, ty = threadIdx.y;
  __shared__ float ssum[4][64], smax[4][64];
  float sum = 0.f, mx = -FLT_MAX;
  if (c < C) {
    float sc = 0.f, bi = 0.f;
    if constexpr (PRO) { sc = pro.scale[c]; bi = pro.bias[c]; }
    for (int p = ty; p < HW; p += 4) {
      float v = x[((size_t)b * HW + p) * ldx + coff + c];
      const float mk = pro.mask[(size_t)b * HW + p];
      if constexpr (PRO) v = act_f<ACT>(v * sc + bi) * mk;
      sum += v;
      if constexpr (!VALUE) mx = fmaxf(mx, v + (mk * 1e4f - 1e4f));
    }
  }
  ssum[ty][threadIdx.x] = sum;
  smax[ty][threadIdx.x] = mx;
  __syncthreads();
  if (ty == 0 && c < C) {
    const float s = (ssum[0][threadIdx.x] + ssum[1][threadIdx.x]) + (ssum[2][threadIdx.x] + ssum[3][threadIdx.x]);
    const float mean = s / area[b];
    float* o = out + (size_t)b * 3 * C;
    o[c] = mean;
    o[C + c] = mean * s1[b];
    if constexpr (VALUE) o[2 * C + c] = mean * s2[b];
    else o[2 * C + c] = fmaxf(fmaxf(smax[0][threadIdx.x], smax[1][threadIdx.x]), fmaxf(smax[2][threadIdx.x], smax[3][threadIdx.x]));
  }
}

void launch_pool(const float* x, int ldx, int coff, int C, const Prologue& pro, const float* area, const float* s1,
                 const float* s2, bool value, float* out, int B, hipStream_t s) {
  dim3 grid((C + 63) / 64, B), block(64, 4);
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
// Small matmuls (global inputs, pooled features, value head): one thread per (row, output)
// ---------------------------------------------------------------------------------------------------------

template <int ACT>
__global__ __launch_bounds__(64) void small_mm_kernel(const float* __restrict__ in, int ldin, int IC,
                                                      const float* __restrict__ W, int OC, const float* __restrict__ bias,
                                                      float* __restrict__ out, long ldout, int ostride, int accumulate) {
  const int o = blockIdx.x * 64 + threadIdx.x, b = blockIdx.y;
  if (o >= OC) return;
  const float* xr = in + (size_t)b * ldin;
  float acc = 0.f;
  for (int i = 0; i < IC; i++) acc += xr[i] * W[(size_t)i * OC + o];
  if (bias) acc += bias[o];
  acc = act_f<ACT>(acc);
  float* p = out + (size_t)b * ldout + (size_t)o * ostride;
  *p = accumulate ? *p + acc : acc;
}

void launch_small_matmul(const float* in, int ldin, int IC, const float* W, int OC, const float* bias, int act,
                         float* out, long ldout, int ostride, bool accumulate, int B, hipStream_t s) {
  dim3 grid((OC + 63) / 64, B);
  const int a = accumulate ? 1 : 0;
  switch (act) {
    case ACT_RELU: small_mm_kernel<ACT_RELU><<<grid, 64, 0, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
    case ACT_MISH: small_mm_kernel<ACT_MISH><<<grid, 64, 0, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
    case ACT_SILU: small_mm_kernel<ACT_SILU><<<grid, 64, 0, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
    default: small_mm_kernel<ACT_ID><<<grid, 64, 0, s>>>(in, ldin, IC, W, OC, bias, out, ldout, ostride, a); break;
  }
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Head: policy p2 conv and ownership conv per board point, written into the readback rows
// ---------------------------------------------------------------------------------------------------------

template <int PACT, int VACT>
__global__ __launch_bounds__(64) void head_spatial_kernel(HeadSpatialArgs a) {
  const int pos = blockIdx.x * 64 + threadIdx.x, b = blockIdx.y;
  if (pos >= HW) return;
  const size_t m = (size_t)b * HW + pos;
  const float* h = a.H + m * a.ldh;
  const float mk = a.mask[m];
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
  dim3 grid((HW + 63) / 64, B);
  if (a.p1_act != a.v1_act) throw std::runtime_error("head: p1 and v1 activations differ");
  switch (a.p1_act) {
    case ACT_RELU: head_spatial_kernel<ACT_RELU, ACT_RELU><<<grid, 64, 0, s>>>(a); break;
    case ACT_MISH: head_spatial_kernel<ACT_MISH, ACT_MISH><<<grid, 64, 0, s>>>(a); break;
    case ACT_SILU: head_spatial_kernel<ACT_SILU, ACT_SILU><<<grid, 64, 0, s>>>(a); break;
    default: head_spatial_kernel<ACT_ID, ACT_ID><<<grid, 64, 0, s>>>(a); break;
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
