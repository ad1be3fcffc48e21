// MFMA GEMM for gfx950: C[z][m][n] = sum_k A[z][m][k] * Bt[z][n][k] with float accumulation
// (v_mfma_f32_16x16x32_{f16,bf16}, v_mfma_f32_16x16x4_f32). Serves the 1x1 convolutions, the F(4x4,3x3) point
// GEMMs, the transformer linears and the head's first convolutions; its epilogue is conv_store (bias, board mask,
// compute-type store, float store or residual add, and emission of the next consumer's activation).
#include "kgx_device.h"

#include <climits>

namespace kgx {

// Cfg: BM x BN output tile per workgroup of WM x WN waves, each wave (BM/WM) x (BN/WN) built from
// 16x16 MFMA blocks. K advances BK at a time (several MFMA K steps), so each stage moves tens of KB: the next
// stage's global loads are in flight in registers while the current stage, double-buffered in LDS with a 16-byte
// row pad, feeds the MFMAs; one barrier per stage. A may be float (the head's f32 trunk): a BN + activation + mask
// prologue then runs as the stage is written to LDS and values are converted to T there.
template <int BM_, int BN_, int BKH_, int WM_, int WN_, bool KFULL_ = false, int MINW_ = 2>
struct Cfg {
  static constexpr int MINW = MINW_;  // waves per SIMD the register allocation must allow
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int BKH = BKH_;  // K per stage for 16-bit types (float uses half as many)
  // K is a multiple of the stage depth (the dispatcher checks): loads need no K bound, and rows past M or N are
  // clamped to the last one instead of zeroed, since they only feed outputs that are not stored.
  static constexpr bool KFULL = KFULL_;
};

// Epilogue variants, chosen at launch so that a kernel carries only its own epilogue code (a kernel holding all
// of them ran 15-25 % slower on the token GEMMs, its main loop unchanged).
enum GemmEpi {
  EPI_SCALAR,  // per-element conv_store (rows or columns not 16-byte aligned)
  EPI_GEN,     // conv_store4: any of colbias, rowmask, yt, y (+ residual), emission
  EPI_YT,      // compute-type store only
  EPI_ACC,     // float store or residual add (+ row mask) only
  EPI_GLU,     // gated output
  EPI_QKV,     // q|k|v projection
  EPI_YTMISH,  // compute-type store of mish(C)
};

// Tile order. Workgroup g runs on XCD g % 8, and each XCD owns every eighth row tile (row tile r on XCD r % 8):
// the row tile's A rows are fetched into one L2 and read there by all its column tiles, and the cache lines that
// neighbouring column tiles share in the output meet in that L2. An XCD walks its column tiles in chunks of `cn`
// tiles whose slice of B (cn x BN x K operands) takes at most 2 MB of its 4 MB L2: for each chunk, each of its row
// tiles with every column tile of the chunk. When all of B fits (cn = all column tiles), each XCD keeps all of B.
// Against the column-fastest order (each XCD an eighth of the column tiles, every row tile's A in all eight L2s):
// b10c384h6 at batch 32 1.387 -> 1.29 ms per forward, b10c512h8 and tf3-b11c768 at batch 64 3.907 -> 3.73 and
// 7.68 -> 7.63 ms; 1 MB chunks were slower than 2 MB on all three. Ids past the last row tile (the row tiles are
// rounded up to 8) exit at once.
__host__ __device__ inline int gemm_chunk(int ntn, int BN, int K, int tsize) {
  const long tile_b = (long)BN * K * tsize;
  int cn = (int)(2048l * 1024 / tile_b);
  if (cn >= ntn) return ntn;
  if (cn < 1) cn = 1;
  while (ntn % cn) cn--;  // a divisor of the column tiles, so that every chunk is whole
  return cn;
}
__host__ __device__ inline void gemm_tile_of(int g, int ntm, int ntn, int cn, int& mt, int& nt) {
  const int rm = (ntm + 7) / 8, slot = g >> 3, per = rm * cn;
  const int j = slot / per, rem = slot - j * per, r = rem / cn;
  nt = j * cn + (rem - r * cn);
  mt = (g & 7) + 8 * r;
}
__host__ inline int gemm_grid(int M, int N, int BM, int BN) {
  return 8 * (((M + BM - 1) / BM + 7) / 8) * ((N + BN - 1) / BN);
}

// The rotation of x with its partner y (the other half of the head): x cos - y sin for the first half, y sin + x cos
// for the second, each with one explicit fused multiply-add, so that every tile configuration rounds it alike (a
// contracted expression may fuse either product, and a row must not depend on the tile it falls in).
__device__ __forceinline__ floatx4 rope4(floatx4 x, floatx4 y, floatx4 cs, floatx4 sn, bool lo) {
  floatx4 r;
#pragma unroll
  for (int k = 0; k < 4; k++)
    r[k] = lo ? __builtin_fmaf(x[k], cs[k], -(y[k] * sn[k])) : __builtin_fmaf(y[k], sn[k], x[k] * cs[k]);
  return r;
}

template <typename T, typename C, bool AF, bool PRO, int ACT, int EPI>
// The operands' pointers, strides and sizes lead the arguments (copies of g's fields) so that they are preloaded
// into SGPRs at wave launch; by-value structs are not, and the first stage's loads would wait for them.
__global__ __launch_bounds__(C::WM * C::WN * 64, C::MINW) void gemm_kernel(const void* gA, const void* gBt, long sA,
                                                                          long sB, int M, int N, int K, int lda,
                                                                          int ldb, GemmArgs g) {
  constexpr int BM = C::BM, BN = C::BN, WM = C::WM, WN = C::WN, NT = WM * WN * 64;
  constexpr int VEC = Tile<T>::VEC;
  constexpr int BK = sizeof(T) == 2 ? C::BKH : C::BKH / 2;
  // 128-byte rows (16-bit, BK = 64) are stored unpadded with their 16-byte chunks swizzled (chunk ^ (row/2 % 8)):
  // the 16 rows x 4 chunks of a fragment read then hit distinct banks. Other widths pad rows by 16 bytes.
  constexpr bool SWZ = sizeof(T) == 2 && BK == 64;
  constexpr int LDK = SWZ ? BK : BK + VEC;
  constexpr int KV = BK / VEC;                       // 16-byte vectors per tile row
  constexpr int AV = BM * KV / NT, BV = BN * KV / NT;
  static_assert(AV * NT == BM * KV && BV * NT == BN * KV, "tile not divisible over the threads");
  constexpr int WTM = BM / WM, WTN = BN / WN;        // wave tile
  constexpr int MB = WTM / 16, NB = WTN / 16;        // MFMA blocks per wave
  constexpr int KS = sizeof(T) == 2 ? 32 : 4;        // K per MFMA
  constexpr int ELD = BN + 4;                        // epilogue float tile row stride
  constexpr int STAGE = 2 * (BM + BN) * LDK * (int)sizeof(T);
  // The epilogue's float tile goes through LDS in EP passes of PR rows (whole wave rows) that fit the stage space.
  constexpr int EP = BM * ELD * 4 <= STAGE || WM == 1 ? 1 : ((BM / 2) * ELD * 4 <= STAGE || WM == 2 ? 2 : 4);
  constexpr int PR = BM / EP, EPIB = PR * ELD * 4;
  static_assert(WM % EP == 0, "epilogue passes split the wave rows");
  __shared__ __align__(1024) char smem[STAGE > EPIB ? STAGE : EPIB];  // 1 KB: each direct-to-LDS load fills one aligned KB
  T (*As)[BM * LDK] = (T (*)[BM * LDK])smem;
  T (*Bs)[BN * LDK] = (T (*)[BN * LDK])(smem + 2 * BM * LDK * sizeof(T));
  typedef u32x4 vec_t;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int z = blockIdx.z;
  int mt, nt;
  {
    const int ntn = (N + BN - 1) / BN;
    gemm_tile_of(blockIdx.x, (M + BM - 1) / BM, ntn, gemm_chunk(ntn, BN, K, (int)sizeof(T)), mt, nt);
  }
  if (mt * BM >= M) return;
  const int n0 = nt * BN, m0 = mt * BM;

  const T* At = (const T*)gA + (size_t)z * sA;
  const float* Af = (const float*)gA + (size_t)z * sA;
  const T* Bt = (const T*)gBt + (size_t)z * sB;

  // Thread-invariant parts of the staged vectors' addresses; per stage only the uniform K offset moves.
  int a_row[AV], a_kk[AV], a_s[AV], b_row[BV], b_kk[BV], b_s[BV];
#pragma unroll
  for (int v = 0; v < AV; v++) {
    const int idx = tid + NT * v;
    a_row[v] = idx / KV;
    a_kk[v] = (idx % KV) * VEC;
    a_s[v] = a_row[v] * LDK + (SWZ ? ((a_kk[v] / VEC) ^ ((a_row[v] >> 1) & 7)) * VEC : a_kk[v]);
  }
#pragma unroll
  for (int v = 0; v < BV; v++) {
    const int idx = tid + NT * v;
    b_row[v] = idx / KV;
    b_kk[v] = (idx % KV) * VEC;
    b_s[v] = b_row[v] * LDK + (SWZ ? ((b_kk[v] / VEC) ^ ((b_row[v] >> 1) & 7)) * VEC : b_kk[v]);
  }
  const T* At0 = At + (size_t)m0 * lda;
  const float* Af0 = Af + (size_t)m0 * lda;
  const T* Bt0 = Bt + (size_t)n0 * ldb;
  int a_off[AV], b_off[BV];  // clamped-row offsets (KFULL)
#pragma unroll
  for (int v = 0; v < AV; v++) a_off[v] = min(a_row[v], M - 1 - m0) * lda + a_kk[v];
#pragma unroll
  for (int v = 0; v < BV; v++) b_off[v] = min(b_row[v], N - 1 - n0) * ldb + b_kk[v];

  vec_t ra[AF ? 1 : AV];
  float rf[AF ? AV * VEC : 1];
  vec_t rb[BV];
  // The float-A prologue's per-element parameters travel with the stage's loads (loaded where the A values are,
  // so the stores after the MFMAs wait for no memory).
  constexpr int PV = AF && PRO ? AV : 1;
  float rsc[PV * VEC], rbi[PV * VEC], rpb[PV * VEC], rmk[PV];

  auto load = [&](int k0) {
#pragma unroll
    for (int v = 0; v < AV; v++) {
      if constexpr (!AF && C::KFULL) {
        ra[v] = *(const vec_t*)(At0 + a_off[v] + k0);
        continue;
      }
      const bool ok = m0 + a_row[v] < M && k0 + a_kk[v] < K;
      const int off = ok ? a_row[v] * lda + k0 + a_kk[v] : 0;
      if constexpr (!AF) {
        ra[v] = *(const vec_t*)(At0 + off);
        if (!ok) ra[v] = vec_t{0, 0, 0, 0};
      } else {
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
          float4 q = *(const float4*)(Af0 + off + e);
          if (!ok) q = float4{0.f, 0.f, 0.f, 0.f};
          rf[v * VEC + e] = q.x; rf[v * VEC + e + 1] = q.y; rf[v * VEC + e + 2] = q.z; rf[v * VEC + e + 3] = q.w;
        }
        if constexpr (PRO) {
          const int mm = ok ? m0 + a_row[v] : 0, kc = ok ? k0 + a_kk[v] : 0;
          rmk[v] = g.pro.mask[mm];
#pragma unroll
          for (int e = 0; e < VEC; e++) {
            rsc[v * VEC + e] = g.pro.scale[kc + e];
            rbi[v * VEC + e] = g.pro.bias[kc + e];
          }
          if (g.pro.prebias) {
            const float* pb = g.pro.prebias + (size_t)(mm / HW) * g.pro.ld_prebias + kc;
#pragma unroll
            for (int e = 0; e < VEC; e++) rpb[v * VEC + e] = pb[e];
          }
        }
      }
    }
#pragma unroll
    for (int v = 0; v < BV; v++) {
      if constexpr (C::KFULL) {
        rb[v] = *(const vec_t*)(Bt0 + b_off[v] + k0);
        continue;
      }
      const bool ok = n0 + b_row[v] < N && k0 + b_kk[v] < K;
      const int off = ok ? b_row[v] * ldb + k0 + b_kk[v] : 0;
      rb[v] = *(const vec_t*)(Bt0 + off);
      if (!ok) rb[v] = vec_t{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf, int k0) {
#pragma unroll
    for (int v = 0; v < AV; v++) {
      if constexpr (!AF) {
        *(vec_t*)(&As[buf][a_s[v]]) = ra[v];
      } else {
        T t[VEC];
        if constexpr (PRO) {
          const bool ok = m0 + a_row[v] < M && k0 + a_kk[v] < K;
#pragma unroll
          for (int e = 0; e < VEC; e++) {
            float a = rf[v * VEC + e];
            if (g.pro.prebias) a += rpb[v * VEC + e];
            const float y = act_f<ACT>(a * rsc[v * VEC + e] + rbi[v * VEC + e]) * rmk[v];
            t[e] = to_t<T>(ok ? y : 0.f);
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; e++) t[e] = to_t<T>(rf[v * VEC + e]);
        }
        *(vec_t*)(&As[buf][a_s[v]]) = *(const vec_t*)t;
      }
    }
#pragma unroll
    for (int v = 0; v < BV; v++) *(vec_t*)(&Bs[buf][b_s[v]]) = rb[v];
  };

  floatx4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + BK - 1) / BK;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int koff = sizeof(T) == 2 ? g4 * 8 : g4;
  // Swizzled chunk of this lane's fragment reads: (kk/8 + g4) ^ sw = (kk/8) ^ (g4 ^ sw), kk/8 in {0, 4}.
  const int sw = SWZ ? (g4 ^ ((r16 >> 1) & 7)) : 0;
  // The MFMAs of one stage buffer.
  auto mma = [&](int cur) {
    const T* as = As[cur] + (wm * WTM + r16) * LDK + (SWZ ? 0 : koff);
    const T* bs = Bs[cur] + (wn * WTN + r16) * LDK + (SWZ ? 0 : koff);
    if constexpr (sizeof(T) == 2) {
      // All fragments of the stage are read before its first MFMA, so the later K steps' reads land while the
      // earlier steps compute.
      typedef typename std::conditional<std::is_same<T, f16>::value, half8, bf16x8>::type frag_t;
      constexpr int KST = BK / KS;
      frag_t fa[KST][MB], fb[KST][NB];
#pragma unroll
      for (int q = 0; q < KST; q++) {
        const int ko = SWZ ? ((q * KS / 8) ^ sw) * 8 : q * KS;
#pragma unroll
        for (int i = 0; i < MB; i++) fa[q][i] = *(const frag_t*)(as + i * 16 * LDK + ko);
#pragma unroll
        for (int j = 0; j < NB; j++) fb[q][j] = *(const frag_t*)(bs + j * 16 * LDK + ko);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < KST; q++)
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < NB; j++) {
            if constexpr (std::is_same<T, f16>::value)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[q][i], fb[q][j], acc[i][j], 0, 0, 0);
            else
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[q][i], fb[q][j], acc[i][j], 0, 0, 0);
          }
    } else {
#pragma unroll
      for (int kk = 0; kk < BK; kk += KS)
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < NB; j++) acc[i][j] = mfma16<T>(as + i * 16 * LDK + kk, bs + j * 16 * LDK + kk, acc[i][j]);
    }
  };

  // 16-bit operands with K a multiple of the stage: stages go straight from memory into LDS
  // (buffer_load ... lds, 16 bytes per lane). One instruction fills 8 swizzled 128-byte rows (lane i: row i / 8,
  // stored chunk i % 8, loaded chunk (i % 8) ^ (row / 2 % 8)); the instructions of A and B are dealt round-robin
  // to the waves. Rows past M or N lie beyond the buffer range and read as zero.
  constexpr bool DMA = sizeof(T) == 2 && !AF && C::KFULL && SWZ;
  if constexpr (DMA) {
    constexpr int NW = WM * WN, AI = BM / 8 / NW, BI = BN / 8 / NW;
    static_assert(AI * 8 * NW == BM && BI * 8 * NW == BN, "stage rows not divisible over the waves");
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const long arb = (long)lda * 2, brb = (long)ldb * 2;
    const int abytes = (int)(min(BM, M - m0) * arb), bbytes = (int)(min(BN, N - n0) * brb);
    int aoff[AI], boff[BI];
#pragma unroll
    for (int q = 0; q < AI; q++) {
      const int row = (q * NW + wv) * 8 + (lane >> 3);
      aoff[q] = (int)(row * arb) + (((lane & 7) ^ ((row >> 1) & 7)) * 16);
    }
#pragma unroll
    for (int q = 0; q < BI; q++) {
      const int row = (q * NW + wv) * 8 + (lane >> 3);
      boff[q] = (int)(row * brb) + (((lane & 7) ^ ((row >> 1) & 7)) * 16);
    }
    auto issue = [&](int buf, int k0) {
#pragma unroll
      for (int q = 0; q < AI; q++) lds_load16(At0, abytes, As[buf] + (q * NW + wv) * 8 * LDK, aoff[q] + k0 * 2);
#pragma unroll
      for (int q = 0; q < BI; q++) lds_load16(Bt0, bbytes, Bs[buf] + (q * NW + wv) * 8 * LDK, boff[q] + k0 * 2);
    };
    // Software pipeline over two stage buffers and two fragment register sets: at step kt the fragments of
    // stage kt + 1 are read from LDS while stage kt's MFMAs run, and stage kt + 2 streams into the buffer that
    // stage kt occupied. The compiler does not count these loads, so each wave waits for its own before the
    // barrier (which also waits for the wave's outstanding LDS reads: no buffer is overwritten while read).
    typedef typename std::conditional<std::is_same<T, f16>::value, half8, bf16x8>::type frag_t;
    constexpr int KST = BK / KS;
    frag_t fa[2][KST][MB], fb[2][KST][NB];
    auto rd = [&](int buf, auto setc) {
      constexpr int set = decltype(setc)::value;
      const T* as = As[buf] + (wm * WTM + r16) * LDK;
      const T* bs = Bs[buf] + (wn * WTN + r16) * LDK;
#pragma unroll
      for (int q = 0; q < KST; q++) {
        const int ko = ((q * KS / 8) ^ sw) * 8;
#pragma unroll
        for (int i = 0; i < MB; i++) fa[set][q][i] = *(const frag_t*)(as + i * 16 * LDK + ko);
#pragma unroll
        for (int j = 0; j < NB; j++) fb[set][q][j] = *(const frag_t*)(bs + j * 16 * LDK + ko);
      }
    };
    auto mf = [&](auto setc) {
      constexpr int set = decltype(setc)::value;
#pragma unroll
      for (int q = 0; q < KST; q++)
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < NB; j++) {
            if constexpr (std::is_same<T, f16>::value)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[set][q][i], fb[set][q][j], acc[i][j], 0, 0, 0);
            else
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[set][q][i], fb[set][q][j], acc[i][j], 0, 0, 0);
          }
    };
    // Step kt uses register set kt % 2 and stage buffer kt % 2; the loop runs two steps per trip so that both
    // are compile-time indices (a runtime index would put the register arrays in scratch memory).
    auto step = [&](int kt, auto setc) {
      constexpr int set = decltype(setc)::value;
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (kt + 2 < nk) issue(set, (kt + 2) * BK);
      if (kt + 1 < nk) rd(set ^ 1, std::integral_constant<int, set ^ 1>{});
      mf(setc);
    };
    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    rd(0, std::integral_constant<int, 0>{});
    if (nk > 1) issue(1, BK);
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, std::integral_constant<int, 0>{});
      if (kt + 1 < nk) step(kt + 1, std::integral_constant<int, 1>{});
    }
  } else {
    load(0);
    store(0, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load((kt + 1) * BK);
      mma(cur);
      if (kt + 1 < nk) store(cur ^ 1, (kt + 1) * BK);
      __syncthreads();
    }
  }

  ConvOut o = g.out;
  if (z) {
    if (o.y) o.y += (size_t)z * g.sC;
    if (o.yt) o.yt = (T*)o.yt + (size_t)z * g.sC;
  }
  if constexpr (EPI == EPI_SCALAR) {
    // Output element (i, j, r) of this lane: row wm*WTM + i*16 + 4*(lane/16) + r, column wn*WTN + j*16 + lane%16.
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = m0 + wm * WTM + i * 16 + 4 * (lane >> 4) + r;
          const int nn = n0 + wn * WTN + j * 16 + (lane & 15);
          if (m < M && nn < N) conv_store<T>(o, m, nn, acc[i][j][r]);
        }
    return;
  }
  // Epilogue through LDS (the stage buffers are free after the loop's last barrier), in passes of PR rows: the
  // float tile, then four consecutive columns of one row per thread with 16-byte accesses, the per-row and
  // per-column inputs loaded ahead of the stores.
  float* Et = (float*)smem;
  constexpr int CV = BN / 4, EV = PR * CV / NT;
  static_assert(EV * NT == PR * CV, "epilogue vectors not divisible over the threads");
#pragma unroll
  for (int p = 0; p < EP; p++) {
    if (p) __syncthreads();
    if (wm / (WM / EP) == p) {
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            Et[(wm * WTM - p * PR + i * 16 + 4 * g4 + r) * ELD + wn * WTN + j * 16 + r16] = acc[i][j][r];
    }
    __syncthreads();
    const int mp = m0 + p * PR;
    if constexpr (EPI == EPI_GLU) {
      constexpr int HV = BN / 8;  // 4-wide vectors of gated outputs per tile row
      for (int e = tid; e < PR * HV; e += NT) {
        const int r = e / HV, hc = (e % HV) * 4, lc = (hc / 16) * 32 + hc % 16;
        const int m = mp + r, f = n0 / 2 + hc;
        if (m < M && f < N / 2) {
          const floatx4 a = *(const floatx4*)(Et + r * ELD + lc), b = *(const floatx4*)(Et + r * ELD + lc + 16);
          store4<T>((T*)o.yt + (size_t)m * o.ldyt + f, act_f<ACT_SILU>(a[0]) * b[0], act_f<ACT_SILU>(a[1]) * b[1],
                    act_f<ACT_SILU>(a[2]) * b[2], act_f<ACT_SILU>(a[3]) * b[3]);
        }
      }
    } else if constexpr (EPI == EPI_QKV && NT % CV == 0) {
      // q|k|v projection: each head lies inside the tile, so the rotation partner of column n (n +- dq/2) is
      // in LDS too. A thread keeps one column quad for every row it takes (NT is a multiple of CV), so the head,
      // rotation and table indices are computed once, and the rotation tables are read for all its rows before
      // the first store (a load after a store that may alias it waits for the store).
      constexpr int RS = NT / CV;
      const QkvEpi& q = g.qkv;
      const int half = q.dq / 2;
      const int c = (tid % CV) * 4, n = n0 + c, r0 = tid / CV;
      const bool qk = n < q.nq + q.nk, isq = n < q.nq;
      const int nn = n - (isq ? 0 : q.nq), hh = nn / q.dq, rr = nn - hh * q.dq;
      const bool lo = rr < half;
      const int pp = lo ? rr : rr - half, tab = q.tables == 1 ? 0 : (isq ? hh / (q.H / q.KV) : hh);
      const bool rot = qk && q.cos;
      floatx4 cs[EV], sn[EV];
      if (rot) {
#pragma unroll
        for (int v = 0; v < EV; v++) {
          const int m = min(mp + r0 + RS * v, M - 1);
          const size_t ti = ((size_t)tab * HW + m % HW) * half + pp;
          cs[v] = *(const floatx4*)(q.cos + ti);
          sn[v] = *(const floatx4*)(q.sin + ti);
        }
      }
#pragma unroll
      for (int v = 0; v < EV; v++) {
        const int r = r0 + RS * v, m = mp + r;
        if (m < M && n < N) {
          floatx4 x = *(const floatx4*)(Et + r * ELD + c);
          if (qk) {
            if (rot) {
              const floatx4 y = *(const floatx4*)(Et + r * ELD + c + (lo ? half : -half));
              x = rope4(x, y, cs[v], sn[v], lo);
            }
            if (isq) x *= q.qscale;
          }
          store4<T>((T*)o.yt + (size_t)m * o.ldyt + n, x[0], x[1], x[2], x[3]);
        }
      }
    } else if constexpr (EPI == EPI_QKV) {
      // (The same on tiles whose thread count is not a multiple of their column quads.)
      const QkvEpi& q = g.qkv;
      const int half = q.dq / 2;
#pragma unroll
      for (int v = 0; v < EV; v++) {
        const int e = tid + NT * v, r = e / CV, c = (e % CV) * 4, m = mp + r, n = n0 + c;
        if (m < M && n < N) {
          floatx4 x = *(const floatx4*)(Et + r * ELD + c);
          if (n < q.nq + q.nk) {
            const bool isq = n < q.nq;
            const int hh = (n - (isq ? 0 : q.nq)) / q.dq, rr = (n - (isq ? 0 : q.nq)) - hh * q.dq;
            if (q.cos) {
              const bool lo = rr < half;
              const int pp = lo ? rr : rr - half, tab = q.tables == 1 ? 0 : (isq ? hh / (q.H / q.KV) : hh);
              const floatx4 y = *(const floatx4*)(Et + r * ELD + c + (lo ? half : -half));
              const size_t ti = ((size_t)tab * HW + m % HW) * half + pp;
              const floatx4 cs = *(const floatx4*)(q.cos + ti), sn = *(const floatx4*)(q.sin + ti);
              x = rope4(x, y, cs, sn, lo);
            }
            if (isq) x *= q.qscale;
          }
          store4<T>((T*)o.yt + (size_t)m * o.ldyt + n, x[0], x[1], x[2], x[3]);
        }
      }
    } else if constexpr (EPI == EPI_YT || EPI == EPI_YTMISH) {
#pragma unroll
      for (int v = 0; v < EV; v++) {
        const int e = tid + NT * v, r = e / CV, c = (e % CV) * 4, m = mp + r, n = n0 + c;
        if (m < M && n < N) {
          floatx4 x = *(const floatx4*)(Et + r * ELD + c);
          if constexpr (EPI == EPI_YTMISH) {
#pragma unroll
            for (int q = 0; q < 4; q++) x[q] = sizeof(T) == 2 ? act16<ACT_MISH>(x[q], 1.f) : act_f<ACT_MISH>(x[q]);
          }
          store4<T>((T*)o.yt + (size_t)m * o.ldyt + n, x[0], x[1], x[2], x[3]);
        }
      }
    } else if constexpr (EPI == EPI_ACC) {
      // Float output, the residual and row mask loaded ahead of the stores.
      floatx4 yres[EV];
      float rmv[EV];
#pragma unroll
      for (int v = 0; v < EV; v++) {
        const int e = tid + NT * v, m = min(mp + e / CV, M - 1), n = min(n0 + (e % CV) * 4, N - 4);
        yres[v] = o.accumulate ? *(const floatx4*)(o.y + (size_t)m * o.ldy + n) : floatx4{0.f, 0.f, 0.f, 0.f};
        rmv[v] = o.rowmask ? o.rowmask[m] : 1.f;
      }
#pragma unroll
      for (int v = 0; v < EV; v++) {
        const int e = tid + NT * v, r = e / CV, c = (e % CV) * 4, m = mp + r, n = n0 + c;
        if (m < M && n < N)
          *(floatx4*)(o.y + (size_t)m * o.ldy + n) = *(const floatx4*)(Et + r * ELD + c) * rmv[v] + yres[v];
      }
    } else {
      // Generic (EPI_GEN): one vector at a time, not unrolled, to keep the code small.
#pragma unroll 1
      for (int v = 0; v < EV; v++) {
        const int e = tid + NT * v, r = e / CV, c = (e % CV) * 4, m = mp + r, n = n0 + c;
        if (m < M && n < N) {
          const floatx4 yres = o.y && o.accumulate ? *(const floatx4*)(o.y + (size_t)m * o.ldy + n)
                                                   : floatx4{0.f, 0.f, 0.f, 0.f};
          floatx4 es = {1.f, 1.f, 1.f, 1.f}, eb = {0.f, 0.f, 0.f, 0.f};
          float mk = 1.f;
          if (o.emit.scale) {
            es = *(const floatx4*)(o.emit.scale + n);
            eb = *(const floatx4*)(o.emit.bias + n);
            mk = o.emit.mask[m];
          }
          conv_store4<T>(o, m, n, *(const floatx4*)(Et + r * ELD + c), yres, o.rowmask ? o.rowmask[m] : 1.f, es,
                         eb, mk);
        }
      }
    }
  }
}

// Tile configurations: narrow rows over all of a <= 192-wide N (1x1 convolutions, Winograd point GEMMs: the
// prologue runs once per element), 64x96 for 65..96 columns (the heads), 128x128 for wide GEMMs (transformer
// linears), 64x64 for the rest.
typedef Cfg<32, 192, 64, 1, 4, true> CfgNarrow;
typedef Cfg<128, 128, 64, 2, 2, true> CfgWide;
// 96x96 (three workgroups per CU) for a 16-bit GEMM whose 128x128 grid would not fill two workgroups per CU, or
// whose last round of them would be nearly empty at short K: there the tile's serial chain sets the time, and a
// tile of 56 % of the work shortens it (b10c384h6 at batch 32: N = 384 GEMMs 25.4 against 27.3 us per token
// GEMM on average, +5.4 % end to end; the N = 1536 FFN's third round, +3.4 % more). On grids that fill the chip
// the 128x128 tile's reuse wins (N = 512 and 768 at batch 64: 71.6 against 76.2 us; tf3's K = 768 and 3072
// GEMMs with a nearly empty last round: -1.6 %).
typedef Cfg<96, 96, 64, 2, 2, true, 3> CfgMid;
typedef Cfg<64, 64, 32, 2, 2> CfgSmall;
// 64x128 (three workgroups per CU) for a q|k|v projection whose 128x128 grid is under two rounds of two per CU: the
// tile still holds whole 64-channel heads for the rotation, and half-size tiles even out the rounds (b10c384h6 at
// batch 32: 819 tiles of 128x128 for 512 slots, 30.2 -> 25.6 us, +3.4 % end to end). Measured and rejected: the
// same tile at batch 64 (tf3-b11c768's q|k|v 120.8 -> 124.0 us) and for b10c384h6's other GEMMs in place of 96x96
// (FFN2 27.5 -> 31.9 us).
typedef Cfg<64, 128, 64, 2, 2, true, 3> CfgQkv;
typedef Cfg<64, 96, 64, 2, 2, true> CfgHead;  // the heads' first convolutions: N = p1 + g1 + v1 channels <= 96
// Float operands on the head tile take 64 channels per stage (six stages at 384 channels): 20.8 against 21.8 us
// with 32 at b18c384nbt batch 32. Its 87 KB of LDS allow one workgroup per CU.
typedef Cfg<64, 96, 128, 2, 2, true, 1> CfgHeadF;

// The epilogue a GEMM's outputs need (launch_gemm has set vec_epi and validated glu / qkv).
static int gemm_epi(const GemmArgs& g) {
  const ConvOut& o = g.out;
  if (!g.vec_epi) return EPI_SCALAR;
  if (g.glu) return EPI_GLU;
  if (g.qkv.dq) return EPI_QKV;
  if (g.yt_act == ACT_MISH) return EPI_YTMISH;
  if (o.colbias || o.emit.scale) return EPI_GEN;
  if (o.yt && !o.y && !o.rowmask) return EPI_YT;
  if (o.y && !o.yt && !o.y_dead) return EPI_ACC;
  return EPI_GEN;
}

template <typename T, typename C, bool AF, bool PRO, int ACT>
static void gemm_launch(const GemmArgs& g, hipStream_t s) {
  const int epi = gemm_epi(g);
  if (g.qkv.dq && C::BN % g.qkv.dq)
    throw std::runtime_error("gemm: the q|k|v epilogue needs the column tile to hold whole heads");
  dim3 grid(gemm_grid(g.M, g.N, C::BM, C::BN), 1, g.Z);
  if (g.lda > INT_MAX || g.ldb > INT_MAX) throw std::runtime_error("gemm: row stride beyond the int range");
  auto go = [&](auto kernel) {
    launch_k(kernel, grid, C::WM * C::WN * 64, 0, s, g.A, g.Bt, g.sA, g.sB, g.M, g.N, g.K, (int)g.lda, (int)g.ldb, g);
  };
  switch (epi) {
    case EPI_SCALAR: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_SCALAR>); break;
    case EPI_YT: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_YT>); break;
    case EPI_ACC: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_ACC>); break;
    case EPI_GLU: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_GLU>); break;
    case EPI_QKV: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_QKV>); break;
    case EPI_YTMISH: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_YTMISH>); break;
    default: go(gemm_kernel<T, C, AF, PRO, ACT, EPI_GEN>); break;
  }
}

// The tile a GEMM runs on (gemm_cfg launches it; gemm_row_tile reports its rows).
enum GemmTile { GT_HEADF, GT_HEAD, GT_NARROW, GT_MID, GT_QKV, GT_WIDE, GT_SMALL };
static GemmTile gemm_tile_choice(const GemmArgs& g, int tsize, bool af) {
  const int bkh = 64, bk = tsize == 2 ? bkh : bkh / 2;
  if (g.N > 64 && g.N <= 96 && g.K % 64 == 0 && tsize == 4) return GT_HEADF;
  if (g.N > 64 && g.N <= 96 && g.K % bk == 0) return GT_HEAD;
  if (g.N > 128 && g.N <= 192 && g.K % bk == 0) return GT_NARROW;
  if (g.N > 192 && g.N <= 384 && g.K % bk == 0 && af) return GT_NARROW;
  if (af) return GT_SMALL;  // (float-A prologue kernels are not built on the wide tile: their staging registers spill there)
  if (tsize == 2) {
    // Also when a short-K GEMM's last round of 128x128 tiles would be under a quarter full.
    const long wide_tiles = (long)((g.M + 127) / 128) * ((g.N + 127) / 128);
    const bool tail = (wide_tiles % 512) * 4 < 512 && g.K <= 512;
    if (g.N > 128 && g.K % bk == 0 && !g.qkv.dq && g.Z == 1 && (wide_tiles < 512 || tail)) return GT_MID;
    if (g.qkv.dq && g.N > 128 && g.K % bk == 0 && g.Z == 1 && wide_tiles < 1024) return GT_QKV;
    // Also for a GEMM whose 128x128 grid is under three rounds with its last round under half full (the batch-64
    // nets' N = 512 and 768 out projections and FFN2: b10c512h8 out 35.2 -> 31.5 us, +0.9 % end to end; tf3-b11c768
    // FFN2 173.6 -> 167.3 us, out 65.9 -> 60.5, +0.5 %).
    const long last = wide_tiles % 512;
    if (!g.qkv.dq && g.N > 128 && g.K % bk == 0 && g.Z == 1 && wide_tiles < 3 * 512 && last > 0 && 2 * last < 512)
      return GT_QKV;
  }
  if (g.N > 128 && g.K % bk == 0 && (long)((g.M + 127) / 128) * ((g.N + 127) / 128) * g.Z >= 256) return GT_WIDE;
  return GT_SMALL;
}

int gemm_row_tile(int prec, int M, int N, int K) {
  GemmArgs g;
  g.M = M; g.N = N; g.K = K;
  switch (gemm_tile_choice(g, prec == PREC_F32 ? 4 : 2, false)) {
    case GT_HEADF: return CfgHeadF::BM;
    case GT_HEAD: return CfgHead::BM;
    case GT_NARROW: return CfgNarrow::BM;
    case GT_MID: return CfgMid::BM;
    case GT_QKV: return CfgQkv::BM;
    case GT_WIDE: return CfgWide::BM;
    default: return CfgSmall::BM;
  }
}

template <typename T, bool AF, bool PRO, int ACT>
static void gemm_cfg(const GemmArgs& g, hipStream_t s) {
  switch (gemm_tile_choice(g, (int)sizeof(T), AF)) {
    case GT_HEADF:
      if constexpr (sizeof(T) == 4) gemm_launch<T, CfgHeadF, AF, PRO, ACT>(g, s);  // (built for float only)
      break;
    case GT_HEAD: gemm_launch<T, CfgHead, AF, PRO, ACT>(g, s); break;
    case GT_NARROW: gemm_launch<T, CfgNarrow, AF, PRO, ACT>(g, s); break;
    case GT_MID:
      if constexpr (sizeof(T) == 2 && !AF) gemm_launch<T, CfgMid, AF, PRO, ACT>(g, s);
      break;
    case GT_QKV:
      if constexpr (sizeof(T) == 2 && !AF) gemm_launch<T, CfgQkv, AF, PRO, ACT>(g, s);
      break;
    case GT_WIDE:
      if constexpr (!AF) gemm_launch<T, CfgWide, AF, PRO, ACT>(g, s);
      break;
    default: gemm_launch<T, CfgSmall, AF, PRO, ACT>(g, s); break;
  }
}

template <typename T>
static void gemm_t(const GemmArgs& g, hipStream_t s) {
  if (!g.a_float) {
    gemm_cfg<T, false, false, ACT_ID>(g, s);
  } else if (!g.pro.scale) {
    gemm_cfg<T, true, false, ACT_ID>(g, s);
  } else {
    switch (g.pro.act) {
      case ACT_RELU: gemm_cfg<T, true, true, ACT_RELU>(g, s); break;
      case ACT_MISH: gemm_cfg<T, true, true, ACT_MISH>(g, s); break;
      case ACT_SILU: gemm_cfg<T, true, true, ACT_SILU>(g, s); break;
      default: gemm_cfg<T, true, true, ACT_ID>(g, s); break;
    }
  }
}

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Whether the four-column vector epilogue applies: every output row and column block it touches is 16-byte
// (float) / 8-byte (16-bit) aligned.
static bool vector_epilogue_ok(const GemmArgs& g, int tsize) {
  const ConvOut& o = g.out;
  if (g.N % 4 || (g.Z > 1 && g.sC % 4)) return false;
  if (o.y && (o.ldy % 4 || !aligned(o.y, 16))) return false;
  if (o.yt && (o.ldyt % 4 || !aligned(o.yt, 4 * tsize))) return false;
  if (o.colbias && (o.ld_colbias % 4 || !aligned(o.colbias, 16))) return false;
  if (o.emit.scale && (o.emit.ld % 4 || !aligned(o.emit.out, 4 * tsize) || !aligned(o.emit.scale, 16) ||
                       !aligned(o.emit.bias, 16)))
    return false;
  return true;
}

void launch_gemm(int prec, const GemmArgs& g0, hipStream_t s) {
  if (g0.M <= 0 || g0.N <= 0 || g0.K <= 0) return;
  const int vec = prec == PREC_F32 ? 4 : 8;
  if (g0.K % vec != 0 || g0.lda % vec != 0 || g0.ldb % vec != 0)
    throw std::runtime_error("gemm: K and strides must be multiples of the vector width");
  if (g0.Z > 1 && g0.out.emit.scale) throw std::runtime_error("gemm: batched GEMMs carry no emission");
  GemmArgs g = g0;
  g.vec_epi = vector_epilogue_ok(g, prec == PREC_F32 ? 4 : 2);
  if (g.yt_act != ACT_ID) {
    const ConvOut& o = g.out;
    if (g.yt_act != ACT_MISH || !g.vec_epi || g.glu || g.qkv.dq || !o.yt || o.y || o.emit.scale || o.colbias ||
        o.rowmask)
      throw std::runtime_error("gemm: an output activation needs only a compute-type store (mish)");
  }
  if (g.qkv.dq) {
    const ConvOut& o = g.out;
    const QkvEpi& q = g.qkv;
    if (!g.vec_epi || g.glu || g.Z != 1 || !o.yt || o.y || o.emit.scale || o.colbias || o.rowmask || q.dq % 8 ||
        q.nq % q.dq || q.nk % q.dq || q.H < 1 || q.KV < 1 || q.H % q.KV ||
        (q.cos && (!q.sin || !aligned(q.cos, 16) || !aligned(q.sin, 16))))
      throw std::runtime_error("gemm: bad q|k|v epilogue arguments");
  }
  if (g.glu) {
    const ConvOut& o = g.out;
    if (!g.vec_epi || g.N % 32 || g.Z != 1 || !o.yt || o.y || o.emit.scale || o.colbias || o.rowmask)
      throw std::runtime_error("gemm: the gated output needs N % 32 == 0, one GEMM and only a compute-type store");
  }
  if (prec == PREC_F16) gemm_t<f16>(g, s);
  else if (prec == PREC_BF16) gemm_t<bf16>(g, s);
  else gemm_t<float>(g, s);
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
