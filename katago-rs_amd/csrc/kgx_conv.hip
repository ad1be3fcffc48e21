// Convolution kernels for gfx950: Winograd F(4x4,3x3) (the reference's algorithm) and F(2x2,3x3) transforms, the
// F(2x2,3x3) point GEMMs fused with the output transform on MFMA, and a direct odd-k convolution.
//
// Inputs are the consumer activations that the producing layer's epilogue writes (act(BN(x)) * mask in the compute
// type), so no batch norm or activation is recomputed here; outputs go through conv_store (bias, residual, float
// store, emission of the next consumer's activation).
//
// F(4x4,3x3) follows crates/katago-nn-burn/src/wino/kernels.rs: tile scatter and input transform :79-179, output
// transform :312-384, filter transform :36-69.
#include "kgx_device.h"

namespace kgx {

// ---------------------------------------------------------------------------------------------------------
// Transform matrices
// ---------------------------------------------------------------------------------------------------------
// F(4x4,3x3): input tile 6x6 every 4 points, B^T rows 4,0,-5,0,1,0 / 0,-4,-4,1,1,0 / 0,4,-4,-1,1,0 /
// 0,-2,-1,2,1,0 / 0,2,-1,-2,1,0 / 0,4,0,-5,0,1 and A^T rows 1,1,1,1,1,0 / 0,1,-1,2,-2,0 / 0,1,1,4,4,0 /
// 0,1,-1,8,-8,1 (wino/kernels.rs:151-156, 352-355). F(2x2,3x3): input tile 4x4 every 2 points, B^T rows
// 1,0,-1,0 / 0,1,1,0 / 0,-1,1,0 / 0,1,0,-1 and A^T rows 1,1,1,0 / 0,1,-1,-1 (Lavin & Gray 2015); its transformed
// values stay within a few times the inputs, which keeps 16-bit GEMM operands accurate.

template <int TM>
__device__ __forceinline__ void bt_apply(const float* z, float* o);
template <>
__device__ __forceinline__ void bt_apply<4>(const float* z, float* o) {
  o[0] = 4.f * z[0] - 5.f * z[2] + z[4];
  o[1] = -4.f * z[1] - 4.f * z[2] + z[3] + z[4];
  o[2] = 4.f * z[1] - 4.f * z[2] - z[3] + z[4];
  o[3] = -2.f * z[1] - z[2] + 2.f * z[3] + z[4];
  o[4] = 2.f * z[1] - z[2] - 2.f * z[3] + z[4];
  o[5] = 4.f * z[1] - 5.f * z[3] + z[5];
}
template <>
__device__ __forceinline__ void bt_apply<2>(const float* z, float* o) {
  o[0] = z[0] - z[2];
  o[1] = z[1] + z[2];
  o[2] = z[2] - z[1];
  o[3] = z[1] - z[3];
}

template <int TM>
__device__ __forceinline__ void at_apply(const float* z, float* o);
template <>
__device__ __forceinline__ void at_apply<4>(const float* z, float* o) {
  o[0] = z[0] + z[1] + z[2] + z[3] + z[4];
  o[1] = (z[1] - z[2]) + 2.f * (z[3] - z[4]);
  o[2] = (z[1] + z[2]) + 4.f * (z[3] + z[4]);
  o[3] = (z[1] - z[2]) + 8.f * (z[3] - z[4]) + z[5];
}
template <>
__device__ __forceinline__ void at_apply<2>(const float* z, float* o) {
  o[0] = z[0] + z[1] + z[2];
  o[1] = z[1] - z[2] - z[3];
}

int wino_tiles(int tm) { return tm == 2 ? Wino<2>::NT : Wino<4>::NT; }
int wino_points(int tm) { return tm == 2 ? Wino<2>::NP : Wino<4>::NP; }

// ---------------------------------------------------------------------------------------------------------
// Input transform
// ---------------------------------------------------------------------------------------------------------
// One workgroup per (row n, band of tile rows, 64 channels). The band's input rows, with the one-point halo of the
// windows, are loaded once (lanes are channels, so loads are coalesced over NHWC rows) into LDS; each (tile,
// channel) transform then reads its window from LDS. Tile t = (n * TX + tile_y) * TX + tile_x; its window starts at
// (TM tile_y - 1, TM tile_x - 1), zero outside the board. Each wave walks board points and tiles that are the same
// for all its lanes, so positions and validity are scalar. V[t][p][c] is written coalesced over channels, a tile's
// points contiguous; channels in [C, c_pad) are written as zeros.
template <int TM>
struct Band {
  static constexpr int R = TM == 2 ? 2 : 1;                // tile rows per band
  static constexpr int NB = (Wino<TM>::TX + R - 1) / R;    // bands per board
  static constexpr int SR = R * TM + 2;                    // staged input rows
  static constexpr int SC = Wino<TM>::TX * TM + 2;         // staged input columns
};

template <typename T, int TM, bool NCHWF32>
__global__ __launch_bounds__(256) void wino_in_kernel(const void* __restrict__ xv, int ldx, T* __restrict__ V, int B,
                                                      int C, int c_pad) {
  using W = Wino<TM>;
  using BD = Band<TM>;
  constexpr int TI = W::TI, NP = W::NP, NS = BD::SR * BD::SC;
  __shared__ float sh[NS * 64];
  const int lane = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.y);
  const int c = blockIdx.x * 64 + lane;
  const int n = blockIdx.y / BD::NB, band = blockIdx.y - n * BD::NB;
  const int y0 = band * BD::R * TM - 1;
  const bool live = c < C;
  const int cl = live ? c : 0;
  // All loads of the unrolled loop are issued from clamped addresses and masked afterwards, so they overlap.
  constexpr int PER = (NS + 3) / 4;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int e = w + 4 * k;
    const int r = e / BD::SC, col = e - r * BD::SC;
    const int yy = y0 + r, xx = col - 1;
    const bool ok = e < NS && (unsigned)yy < (unsigned)POS && (unsigned)xx < (unsigned)POS;
    const int pos = ok ? yy * POS + xx : 0;
    float v;
    if constexpr (NCHWF32) v = ((const float*)xv)[((size_t)n * C + cl) * HW + pos];
    else v = (float)((const T*)xv + ((size_t)n * HW + pos) * ldx)[cl];
    if (e < NS) sh[e * 64 + lane] = (ok && live) ? v : 0.f;
  }
  __syncthreads();
  if (c >= c_pad) return;
  constexpr int TPB = BD::R * W::TX;  // tiles per band
#pragma unroll
  for (int k = 0; k < (TPB + 3) / 4; k++) {
    const int ti = w + 4 * k;
    const int tr = band * BD::R + ti / W::TX, tc = ti % W::TX;
    if (ti >= TPB || tr >= W::TX) break;
    const float* win = sh + ((tr - band * BD::R) * TM * BD::SC + tc * TM) * 64 + lane;
    float d[NP];
#pragma unroll
    for (int sy = 0; sy < TI; sy++)
#pragma unroll
      for (int sx = 0; sx < TI; sx++) d[sy * TI + sx] = win[(sy * BD::SC + sx) * 64];
    float r[NP];
#pragma unroll
    for (int sy = 0; sy < TI; sy++) bt_apply<TM>(&d[sy * TI], &r[sy * TI]);
#pragma unroll
    for (int sx = 0; sx < TI; sx++) {
      float col[TI], o[TI];
#pragma unroll
      for (int j = 0; j < TI; j++) col[j] = r[j * TI + sx];
      bt_apply<TM>(col, o);
#pragma unroll
      for (int j = 0; j < TI; j++) d[j * TI + sx] = o[j];
    }
    const int t = (n * W::TX + tr) * W::TX + tc;
    T* vb = V + (size_t)t * NP * c_pad;
#pragma unroll
    for (int p = 0; p < NP; p++) (vb + p * c_pad)[c] = to_t<T>(d[p]);
  }
}

template <typename T, int TM>
static void wino_in_t(const void* x, int ldx, bool nchw_f32, T* V, int B, int C, int c_pad, hipStream_t s) {
  dim3 block(64, 4), grid((c_pad + 63) / 64, B * Band<TM>::NB);
  if (nchw_f32) launch_k(wino_in_kernel<T, TM, true>, grid, block, 0, s, x, ldx, V, B, C, c_pad);
  else launch_k(wino_in_kernel<T, TM, false>, grid, block, 0, s, x, ldx, V, B, C, c_pad);
}

void launch_wino_in(int prec, int tm, const void* x, int ldx, bool nchw_f32, void* V, int B, int C, int c_pad,
                    hipStream_t s) {
  if (c_pad < C || c_pad % 8 != 0) throw std::runtime_error("wino_in: bad channel padding");
  if (tm != 2 && tm != 4) throw std::runtime_error("wino_in: tile must be 2 or 4");
#define KGX_WI(T) \
  if (tm == 4) wino_in_t<T, 4>(x, ldx, nchw_f32, (T*)V, B, C, c_pad, s); \
  else wino_in_t<T, 2>(x, ldx, nchw_f32, (T*)V, B, C, c_pad, s);
  if (prec == PREC_F16) { KGX_WI(f16) }
  else if (prec == PREC_BF16) { KGX_WI(bf16) }
  else { KGX_WI(float) }
#undef KGX_WI
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Output transform (unfused path): M[t][p][oc] -> conv_store
// ---------------------------------------------------------------------------------------------------------

template <typename T, int TM>
__global__ __launch_bounds__(256) void wino_out_kernel(const float* __restrict__ M, int oc_pad, int OC, ConvOut o,
                                                       int B) {
  using W = Wino<TM>;
  constexpr int TI = W::TI, NP = W::NP;
  const int oc = blockIdx.x * 64 + threadIdx.x;
  const int t = blockIdx.y * 4 + threadIdx.y;
  if (oc >= OC || t >= B * W::NT) return;
  float m[NP];
  const float* mb = M + (size_t)t * NP * oc_pad + oc;
#pragma unroll
  for (int p = 0; p < NP; p++) m[p] = mb[(size_t)p * oc_pad];
  float r[TI * TM];  // [TI rows][TM]
#pragma unroll
  for (int sy = 0; sy < TI; sy++) at_apply<TM>(&m[sy * TI], &r[sy * TM]);
  float out[TM * TM];
#pragma unroll
  for (int sx = 0; sx < TM; sx++) {
    float col[TI], c4[TM];
#pragma unroll
    for (int k = 0; k < TI; k++) col[k] = r[k * TM + sx];
    at_apply<TM>(col, c4);
#pragma unroll
    for (int k = 0; k < TM; k++) out[k * TM + sx] = c4[k];
  }
  const int n = t / W::NT, tile = t - n * W::NT;
  const int ty = tile / W::TX, tx = tile - ty * W::TX;
#pragma unroll
  for (int sy = 0; sy < TM; sy++)
#pragma unroll
    for (int sx = 0; sx < TM; sx++) {
      const int yy = ty * TM + sy, xx = tx * TM + sx;
      if (yy < POS && xx < POS) conv_store<T>(o, n * HW + yy * POS + xx, oc, out[sy * TM + sx]);
    }
}

void launch_wino_out(int prec, int tm, const float* M, int oc_pad, int OC, const ConvOut& o, int B, hipStream_t s) {
  dim3 block(64, 4), grid((OC + 63) / 64, (B * wino_tiles(tm) + 3) / 4);
#define KGX_WO(T) \
  if (tm == 4) launch_k(wino_out_kernel<T, 4>, grid, block, 0, s, M, oc_pad, OC, o, B); \
  else launch_k(wino_out_kernel<T, 2>, grid, block, 0, s, M, oc_pad, OC, o, B);
  if (prec == PREC_F16) { KGX_WO(f16) }
  else if (prec == PREC_BF16) { KGX_WO(bf16) }
  else { KGX_WO(float) }
#undef KGX_WO
  KGX_CHECK_LAUNCH();
}

// Filter transform in double, rounded once to float: U[p][o][i] = (G g G^T)[p]. F(4x4,3x3): G rows (1/4, 0, 0),
// (-1/6, -1/6, -1/6), (-1/6, 1/6, -1/6), (1/24, 1/12, 1/6), (1/24, -1/12, 1/6), (0, 0, 1) (wino/kernels.rs:39-48).
// F(2x2,3x3): G rows (1, 0, 0), (1/2, 1/2, 1/2), (1/2, -1/2, 1/2), (0, 0, 1). Padding is zero.
void wino_filter_host(int tm, const float* w, int oc, int ic, int oc_pad, int ic_pad, float* U) {
  const int ti = tm + 2, np = ti * ti;
  auto g6 = [&](const double z[3], double* o) {
    if (tm == 4) {
      o[0] = 0.25 * z[0];
      o[1] = (-z[0] - z[1] - z[2]) / 6.0;
      o[2] = (-z[0] + z[1] - z[2]) / 6.0;
      o[3] = (z[0] + 2.0 * z[1] + 4.0 * z[2]) / 24.0;
      o[4] = (z[0] - 2.0 * z[1] + 4.0 * z[2]) / 24.0;
      o[5] = z[2];
    } else {
      o[0] = z[0];
      o[1] = (z[0] + z[1] + z[2]) * 0.5;
      o[2] = (z[0] - z[1] + z[2]) * 0.5;
      o[3] = z[2];
    }
  };
  for (size_t k = 0; k < (size_t)np * oc_pad * ic_pad; k++) U[k] = 0.f;
  for (int o = 0; o < oc; o++)
    for (int i = 0; i < ic; i++) {
      double g[9];
      for (int k = 0; k < 9; k++) g[k] = w[((size_t)o * ic + i) * 9 + k];
      double rows[3][6];
      for (int y = 0; y < 3; y++) g6(&g[3 * y], rows[y]);
      for (int xx = 0; xx < ti; xx++) {
        double col[3] = {rows[0][xx], rows[1][xx], rows[2][xx]}, t6[6];
        g6(col, t6);
        for (int y = 0; y < ti; y++) U[(((size_t)(y * ti + xx)) * oc_pad + o) * ic_pad + i] = (float)t6[y];
      }
    }
}

// ---------------------------------------------------------------------------------------------------------
// Fused F(2x2,3x3) GEMM + output transform
// ---------------------------------------------------------------------------------------------------------
// For a block of TB tiles x 64 output channels, the 16 tile-point GEMMs M_p = V_p U_p^T run one after another
// through a double-buffered MFMA pipeline (K staged BK at a time, the next stage's loads in flight in registers),
// and as each M_p completes it is folded into the 2x2 output accumulators (out[sy][sx] += A^T[sy][a] A^T[sx][b]
// M_p, p = 4a + b), so M never leaves registers. Waves are 2x2; each wave owns TB/2 tiles x 32 channels.

template <typename T, int TB, int BKH>
__global__ __launch_bounds__(256) void wino2_fused_kernel(const T* __restrict__ V, const T* __restrict__ U, int t_pad,
                                                          int icp, int ocp, int OC, ConvOut o, int B) {
  using W = Wino<2>;
  constexpr int BN = 64;
  constexpr int VEC = Tile<T>::VEC;
  constexpr int BK = sizeof(T) == 2 ? BKH : BKH / 2;
  constexpr int LDK = BK + VEC;
  constexpr int KV = BK / VEC;
  constexpr int AVT = TB * KV, BVT = BN * KV;  // vectors per stage
  constexpr int AV = (AVT + 255) / 256, BV = BVT / 256;
  static_assert(BV * 256 == BVT, "B stage not divisible over 256 threads");
  constexpr int MB = TB / 32;  // MFMA row blocks per wave
  constexpr int KS = sizeof(T) == 2 ? 32 : 4;  // K per MFMA
  __shared__ __align__(16) T As[2][TB * LDK];
  __shared__ __align__(16) T Bs[2][BN * LDK];
  typedef u32x4 vec_t;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int o0 = blockIdx.x * BN, t0 = blockIdx.y * TB;
  const int nk = icp / BK, total = W::NP * nk;
  const int lda = W::NP * icp;  // tile-major V: row stride of one point's matrix

  // Thread-invariant offsets of the staged vectors (global and LDS); per stage only a uniform base moves.
  int a_g[AV], a_s[AV], b_g[BV], b_s[BV];
#pragma unroll
  for (int v = 0; v < AV; v++) {
    const int idx = tid + 256 * v;
    a_g[v] = (idx / KV) * lda + (idx % KV) * VEC;
    a_s[v] = (idx / KV) * LDK + (idx % KV) * VEC;
  }
#pragma unroll
  for (int v = 0; v < BV; v++) {
    const int idx = tid + 256 * v;
    b_g[v] = (idx / KV) * icp + (idx % KV) * VEC;
    b_s[v] = (idx / KV) * LDK + (idx % KV) * VEC;
  }
  vec_t ra[AV], rb[BV];
  auto load = [&](int it) {
    const int p = it / nk, k0 = (it - p * nk) * BK;
    const T* va = V + (size_t)t0 * lda + p * icp + k0;
    const T* ub = U + ((size_t)p * ocp + o0) * icp + k0;
#pragma unroll
    for (int v = 0; v < AV; v++)
      if (AVT % 256 == 0 || tid + 256 * v < AVT) ra[v] = *(const vec_t*)(va + a_g[v]);
#pragma unroll
    for (int v = 0; v < BV; v++) rb[v] = *(const vec_t*)(ub + b_g[v]);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int v = 0; v < AV; v++)
      if (AVT % 256 == 0 || tid + 256 * v < AVT) *(vec_t*)(&As[buf][a_s[v]]) = ra[v];
#pragma unroll
    for (int v = 0; v < BV; v++) *(vec_t*)(&Bs[buf][b_s[v]]) = rb[v];
  };

  floatx4 macc[MB][2], oacc[4][MB][2];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      macc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; q++) oacc[q][i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  load(0);
  store(0);
  __syncthreads();
  const int r16 = lane & 15, g4 = lane >> 4;
  const int koff = sizeof(T) == 2 ? g4 * 8 : g4;
  for (int it = 0; it < total; it++) {
    const int cur = it & 1;
    if (it + 1 < total) load(it + 1);
    const T* as = As[cur] + (wm * (TB / 2) + r16) * LDK + koff;
    const T* bs = Bs[cur] + (wn * 32 + r16) * LDK + koff;
#pragma unroll
    for (int kk = 0; kk < BK; kk += KS)
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) macc[i][j] = mfma16<T>(as + i * 16 * LDK + kk, bs + j * 16 * LDK + kk, macc[i][j]);
    if ((it + 1) % nk == 0) {
      // Point p complete: fold M_p into the outputs with A^T rows (1,1,1,0) and (0,1,-1,-1).
      const int p = it / nk, pa = p >> 2, pb = p & 3;
      const float ca0 = pa < 3 ? 1.f : 0.f, ca1 = pa == 0 ? 0.f : (pa == 1 ? 1.f : -1.f);
      const float cb0 = pb < 3 ? 1.f : 0.f, cb1 = pb == 0 ? 0.f : (pb == 1 ? 1.f : -1.f);
      const float c00 = ca0 * cb0, c01 = ca0 * cb1, c10 = ca1 * cb0, c11 = ca1 * cb1;
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          oacc[0][i][j] += c00 * macc[i][j];
          oacc[1][i][j] += c01 * macc[i][j];
          oacc[2][i][j] += c10 * macc[i][j];
          oacc[3][i][j] += c11 * macc[i][j];
          macc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    if (it + 1 < total) store(cur ^ 1);
    __syncthreads();
  }

  // Output: element (i, j, r) is tile t0 + wm*TB/2 + i*16 + 4*(lane/16) + r, channel o0 + wn*32 + j*16 + lane%16.
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int t = t0 + wm * (TB / 2) + i * 16 + 4 * (lane >> 4) + r;
      if (t >= B * W::NT) continue;
      const int n = t / W::NT, tile = t - n * W::NT;
      const int ty = tile / W::TX, tx = tile - ty * W::TX;
      const int m00 = n * HW + ty * 2 * POS + tx * 2;
      const bool xin = tx * 2 + 1 < POS, yin = ty * 2 + 1 < POS;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int oc = o0 + wn * 32 + j * 16 + (lane & 15);
        if (oc >= OC) continue;
        conv_store<T>(o, m00, oc, oacc[0][i][j][r]);
        if (xin) conv_store<T>(o, m00 + 1, oc, oacc[1][i][j][r]);
        if (yin) conv_store<T>(o, m00 + POS, oc, oacc[2][i][j][r]);
        if (xin && yin) conv_store<T>(o, m00 + POS + 1, oc, oacc[3][i][j][r]);
      }
    }
}

template <typename T, int BKH>
static void wino2_fused_t(const void* V, const void* U, int t_pad, int icp, int ocp, int OC, const ConvOut& o, int B,
                          hipStream_t s) {
  constexpr int TB = 32;
  dim3 grid(ocp / 64, t_pad / TB);
  launch_k(wino2_fused_kernel<T, TB, BKH>, grid, 256, 0, s, (const T*)V, (const T*)U, t_pad, icp, ocp, OC, o, B);
}

template <typename T>
static void wino2_fused_k(const void* V, const void* U, int t_pad, int icp, int ocp, int OC, const ConvOut& o, int B,
                          hipStream_t s) {
  // The whole of K per stage when it is 192 (one stage per tile point), else 64 or 32.
  if (icp % 192 == 0) wino2_fused_t<T, 192>(V, U, t_pad, icp, ocp, OC, o, B, s);
  else if (icp % 64 == 0) wino2_fused_t<T, 64>(V, U, t_pad, icp, ocp, OC, o, B, s);
  else wino2_fused_t<T, 32>(V, U, t_pad, icp, ocp, OC, o, B, s);
}

void launch_wino2_fused(int prec, const void* V, const void* U, int t_pad, int icp, int ocp, int OC, const ConvOut& o,
                        int B, hipStream_t s) {
  if (t_pad % 64 != 0 || ocp % 64 != 0 || icp % 32 != 0 || t_pad < B * Wino<2>::NT)
    throw std::runtime_error("wino2_fused: bad padding");
  if (prec == PREC_F16) wino2_fused_k<f16>(V, U, t_pad, icp, ocp, OC, o, B, s);
  else if (prec == PREC_BF16) wino2_fused_k<bf16>(V, U, t_pad, icp, ocp, OC, o, B, s);
  else wino2_fused_k<float>(V, U, t_pad, icp, ocp, OC, o, B, s);
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Direct odd-k convolution: one thread per (oc, point, row)
// ---------------------------------------------------------------------------------------------------------

template <typename T, bool NCHWF32>
__global__ __launch_bounds__(64) void conv_direct_kernel(const void* __restrict__ xv, int ldx, int IC,
                                                         const float* __restrict__ w, int OC, int ky, int kx, int dy,
                                                         int dx, ConvOut o) {
  const int oc = blockIdx.x * 64 + threadIdx.x;
  const int pos = blockIdx.y, n = blockIdx.z;
  if (oc >= OC) return;
  const int py = pos / POS, px = pos - py * POS;
  const int oy = (ky / 2) * dy, ox = (kx / 2) * dx;
  float acc = 0.f;
  for (int i = 0; i < IC; i++) {
    for (int a = 0; a < ky; a++) {
      const int sy = py + a * dy - oy;
      if (sy < 0 || sy >= POS) continue;
      for (int b = 0; b < kx; b++) {
        const int sx = px + b * dx - ox;
        if (sx < 0 || sx >= POS) continue;
        const int sp = sy * POS + sx;
        const float v = NCHWF32 ? ((const float*)xv)[((size_t)n * IC + i) * HW + sp]
                                : (float)((const T*)xv)[((size_t)n * HW + sp) * ldx + i];
        acc += v * w[(((size_t)i * ky + a) * kx + b) * OC + oc];
      }
    }
  }
  conv_store<T>(o, n * HW + pos, oc, acc);
}

void launch_conv_direct(int prec, const void* x, int ldx, bool nchw_f32, int IC, const float* w, int OC, int ky, int kx,
                        int dy, int dx, const ConvOut& o, int B, hipStream_t s) {
  dim3 grid((OC + 63) / 64, HW, B);
#define KGX_CD(T)                                                                                   \
  if (nchw_f32) launch_k(conv_direct_kernel<T, true>, grid, 64, 0, s, x, ldx, IC, w, OC, ky, kx, dy, dx, o); \
  else launch_k(conv_direct_kernel<T, false>, grid, 64, 0, s, x, ldx, IC, w, OC, ky, kx, dy, dx, o);
  if (prec == PREC_F16) { KGX_CD(f16) }
  else if (prec == PREC_BF16) { KGX_CD(bf16) }
  else { KGX_CD(float) }
#undef KGX_CD
  KGX_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------------------------------------
// Consumer activation of a float tensor (the mid activation of a global-pooling block, whose bias is known only
// after pooling)
// ---------------------------------------------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(256) void bias_act_kernel(const float* __restrict__ x, int ldx, int C,
                                                       const float* __restrict__ prebias, int ldpb,
                                                       const float* __restrict__ scale, const float* __restrict__ bias,
                                                       int act, const float* __restrict__ mask, T* __restrict__ out,
                                                       int ldo, int rows) {
  const int c = blockIdx.x * 64 + threadIdx.x;
  const int m = blockIdx.y * 4 + threadIdx.y;
  if (c >= C || m >= rows) return;
  float a = x[(size_t)m * ldx + c];
  if (prebias) a += prebias[(size_t)(m / HW) * ldpb + c];
  const float z = a * scale[c] + bias[c];
  out[(size_t)m * ldo + c] = to_t<T>(sizeof(T) == 2 ? act16_rt(z, act, mask[m]) : act_rt(z, act) * mask[m]);
}

// Eight channels per thread: two 16-byte loads of x (and of the per-row bias), one 16-byte store of the result.
template <typename T, int ACT>
__global__ __launch_bounds__(256) void bias_act8_kernel(const float* __restrict__ x, int ldx, int C,
                                                        const float* __restrict__ prebias, int ldpb,
                                                        const float* __restrict__ scale,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ mask, T* __restrict__ out, int ldo,
                                                        int rows) {
  const int vpr = C / 8;  // vectors per row
  const long v = (long)blockIdx.x * 256 + threadIdx.x;
  if (v >= (long)rows * vpr) return;
  const int m = (int)(v / vpr), c = (int)(v - (long)m * vpr) * 8;
  const float* xp = x + (size_t)m * ldx + c;
  floatx4 a0 = *(const floatx4*)xp, a1 = *(const floatx4*)(xp + 4);
  if (prebias) {
    const float* pp = prebias + (size_t)(m / HW) * ldpb + c;
    a0 += *(const floatx4*)pp;
    a1 += *(const floatx4*)(pp + 4);
  }
  const floatx4 s0 = *(const floatx4*)(scale + c), s1 = *(const floatx4*)(scale + c + 4);
  const floatx4 b0 = *(const floatx4*)(bias + c), b1 = *(const floatx4*)(bias + c + 4);
  const float mk = mask[m];
  T t[8];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float x0 = a0[e] * s0[e] + b0[e], x1 = a1[e] * s1[e] + b1[e];
    t[e] = to_t<T>(sizeof(T) == 2 ? act16<ACT>(x0, mk) : act_f<ACT>(x0) * mk);
    t[4 + e] = to_t<T>(sizeof(T) == 2 ? act16<ACT>(x1, mk) : act_f<ACT>(x1) * mk);
  }
  *(u32x4*)(out + (size_t)m * ldo + c) = *(const u32x4*)t;
}

template <typename T>
static void bias_act8_launch(const float* x, int ldx, int C, const float* prebias, int ld_prebias, const float* scale,
                             const float* bias, int act, const float* mask, T* out, int ldo, int rows, hipStream_t s) {
  const long n = (long)rows * (C / 8);
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (act) {
    case ACT_RELU: launch_k(bias_act8_kernel<T, ACT_RELU>, grid, 256, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, mask, out, ldo, rows); break;
    case ACT_MISH: launch_k(bias_act8_kernel<T, ACT_MISH>, grid, 256, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, mask, out, ldo, rows); break;
    case ACT_SILU: launch_k(bias_act8_kernel<T, ACT_SILU>, grid, 256, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, mask, out, ldo, rows); break;
    default: launch_k(bias_act8_kernel<T, ACT_ID>, grid, 256, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, mask, out, ldo, rows); break;
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(u32x4* __restrict__ p, size_t n16, unsigned* __restrict__ tail,
                                                       int ntail) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) p[i] = u32x4{0, 0, 0, 0};
  if (blockIdx.x == 0 && (int)threadIdx.x < ntail) tail[threadIdx.x] = 0u;
}

void launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
  if ((uintptr_t)p % 16 || bytes % 4) throw std::runtime_error("fill_zero: 16-byte aligned, whole words only");
  if (!bytes) return;
  const size_t n16 = bytes / 16;
  const int ntail = (int)((bytes % 16) / 4);
  const int blocks = (int)std::min<size_t>(1024, std::max<size_t>(1, (n16 + 255) / 256));
  launch_k(fill_zero_kernel, blocks, 256, 0, s, (u32x4*)p, n16, (unsigned*)((char*)p + n16 * 16), ntail);
  KGX_CHECK_LAUNCH();
}

void launch_bias_act(int prec, const float* x, int ldx, int C, const float* prebias, int ld_prebias, const float* scale,
                     const float* bias, int act, const float* mask, void* out, int ldo, int rows, hipStream_t s) {
  // 16-byte path for 16-bit outputs when every row and channel group is 16-byte aligned.
  const bool vec = (prec == PREC_F16 || prec == PREC_BF16) && C % 8 == 0 && ldx % 4 == 0 && ldo % 8 == 0 &&
                   (!prebias || ld_prebias % 4 == 0) && ((uintptr_t)x | (uintptr_t)out | (uintptr_t)scale |
                                                          (uintptr_t)bias | (uintptr_t)prebias) % 16 == 0;
  if (vec) {
    if (prec == PREC_F16)
      bias_act8_launch<f16>(x, ldx, C, prebias, ld_prebias, scale, bias, act, mask, (f16*)out, ldo, rows, s);
    else
      bias_act8_launch<bf16>(x, ldx, C, prebias, ld_prebias, scale, bias, act, mask, (bf16*)out, ldo, rows, s);
    KGX_CHECK_LAUNCH();
    return;
  }
  dim3 block(64, 4), grid((C + 63) / 64, (rows + 3) / 4);
  if (prec == PREC_F16)
    launch_k(bias_act_kernel<f16>, grid, block, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, act, mask, (f16*)out, ldo, rows);
  else if (prec == PREC_BF16)
    launch_k(bias_act_kernel<bf16>, grid, block, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, act, mask, (bf16*)out, ldo, rows);
  else
    launch_k(bias_act_kernel<float>, grid, block, 0, s, x, ldx, C, prebias, ld_prebias, scale, bias, act, mask, (float*)out, ldo, rows);
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
