// MFMA GEMM for gfx950: C[z][m][n] = sum_k A[z][m][k] * Bt[z][n][k] with float accumulation
// (v_mfma_f32_16x16x32_{f16,bf16}, v_mfma_f32_16x16x4_f32). Serves the 1x1 convolutions, the F(4x4,3x3) point
// GEMMs, the transformer linears and the head's first convolutions; its epilogue is conv_store (bias, board mask,
// compute-type store, float store or residual add, and emission of the next consumer's activation).
#include "kgx_device.h"

namespace kgx {

// Cfg: BM x BN output tile per workgroup of WM x WN waves, each wave (BM/WM) x (BN/WN) built from
// 16x16 MFMA blocks. K advances BK at a time (several MFMA K steps), so each stage moves tens of KB: the next
// stage's global loads are in flight in registers while the current stage, double-buffered in LDS with a 16-byte
// row pad, feeds the MFMAs; one barrier per stage. A may be float (the head's f32 trunk): a BN + activation + mask
// prologue then runs as the stage is written to LDS and values are converted to T there.
template <int BM_, int BN_, int BKH_, int WM_, int WN_, bool KFULL_ = false>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int BKH = BKH_;  // K per stage for 16-bit types (float uses half as many)
  // K is a multiple of the stage depth (the dispatcher checks): loads need no K bound, and rows past M or N are
  // clamped to the last one instead of zeroed, since they only feed outputs that are not stored.
  static constexpr bool KFULL = KFULL_;
};

template <typename T, typename C, bool AF, bool PRO, int ACT>
__global__ __launch_bounds__(C::WM * C::WN * 64) void gemm_kernel(GemmArgs g) {
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
  constexpr int PR = BM / EP, EPI = PR * ELD * 4;
  static_assert(WM % EP == 0, "epilogue passes split the wave rows");
  __shared__ __align__(16) char smem[STAGE > EPI ? STAGE : EPI];
  T (*As)[BM * LDK] = (T (*)[BM * LDK])smem;
  T (*Bs)[BN * LDK] = (T (*)[BN * LDK])(smem + 2 * BM * LDK * sizeof(T));
  typedef u32x4 vec_t;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int z = blockIdx.z;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int M = g.M, N = g.N, K = g.K;

  const T* At = (const T*)g.A + (size_t)z * g.sA;
  const float* Af = (const float*)g.A + (size_t)z * g.sA;
  const T* Bt = (const T*)g.Bt + (size_t)z * g.sB;

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
  const T* At0 = At + (size_t)m0 * g.lda;
  const float* Af0 = Af + (size_t)m0 * g.lda;
  const T* Bt0 = Bt + (size_t)n0 * g.ldb;
  const int lda = (int)g.lda, ldb = (int)g.ldb;
  int a_off[AV], b_off[BV];  // clamped-row offsets (KFULL)
#pragma unroll
  for (int v = 0; v < AV; v++) a_off[v] = min(a_row[v], M - 1 - m0) * lda + a_kk[v];
#pragma unroll
  for (int v = 0; v < BV; v++) b_off[v] = min(b_row[v], N - 1 - n0) * ldb + b_kk[v];

  vec_t ra[AF ? 1 : AV];
  float rf[AF ? AV * VEC : 1];
  vec_t rb[BV];

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
          const int m = m0 + a_row[v], k = k0 + a_kk[v];
          const bool ok = m < M && k < K;
          const int mm = ok ? m : 0, kc = ok ? k : 0;
          const float mk = g.pro.mask[mm];
          const float* pb = g.pro.prebias ? g.pro.prebias + (size_t)(mm / HW) * g.pro.ld_prebias + kc : nullptr;
          const float* sc = g.pro.scale + kc;
          const float* bi = g.pro.bias + kc;
#pragma unroll
          for (int e = 0; e < VEC; e++) {
            float a = rf[v * VEC + e];
            if (pb) a += pb[e];
            const float y = act_f<ACT>(a * sc[e] + bi[e]) * mk;
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
  load(0);
  store(0, 0);
  __syncthreads();
  const int r16 = lane & 15, g4 = lane >> 4;
  const int koff = sizeof(T) == 2 ? g4 * 8 : g4;
  // Swizzled chunk of this lane's fragment reads: (kk/8 + g4) ^ sw = (kk/8) ^ (g4 ^ sw), kk/8 in {0, 4}.
  const int sw = SWZ ? (g4 ^ ((r16 >> 1) & 7)) : 0;
  for (int kt = 0; kt < nk; kt++) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
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
    if (kt + 1 < nk) store(cur ^ 1, (kt + 1) * BK);
    __syncthreads();
  }

  ConvOut o = g.out;
  if (z) {
    if (o.y) o.y += (size_t)z * g.sC;
    if (o.yt) o.yt = (T*)o.yt + (size_t)z * g.sC;
  }
  if (!g.vec_epi) {
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
    if (g.glu) {
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
      continue;
    }
    constexpr int CV = BN / 4, EV = PR * CV / NT;
    static_assert(EV * NT == PR * CV, "epilogue vectors not divisible over the threads");
    if (g.qkv.dq) {
      // q|k|v projection: each head lies inside the tile, so the rotation partner of column n (n +- dq/2) is
      // in LDS too.
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
              const int p = lo ? rr : rr - half, tab = q.tables == 1 ? 0 : (isq ? hh / (q.H / q.KV) : hh);
              const floatx4 y = *(const floatx4*)(Et + r * ELD + c + (lo ? half : -half));
              const size_t ti = ((size_t)tab * HW + m % HW) * half + p;
              const floatx4 cs = *(const floatx4*)(q.cos + ti), sn = *(const floatx4*)(q.sin + ti);
              x = lo ? x * cs - y * sn : y * sn + x * cs;
            }
            if (isq) x *= q.qscale;
          }
          store4<T>((T*)o.yt + (size_t)m * o.ldyt + n, x[0], x[1], x[2], x[3]);
        }
      }
      continue;
    }
    floatx4 yres[EV];
    float rmv[EV], mkv[EV];
#pragma unroll
    for (int v = 0; v < EV; v++) {
      const int e = tid + NT * v, m = min(mp + e / CV, M - 1), n = min(n0 + (e % CV) * 4, N - 4);
      yres[v] = o.y && o.accumulate ? *(const floatx4*)(o.y + (size_t)m * o.ldy + n) : floatx4{0.f, 0.f, 0.f, 0.f};
      rmv[v] = o.rowmask ? o.rowmask[m] : 1.f;
      mkv[v] = o.emit.scale ? o.emit.mask[m] : 1.f;
    }
#pragma unroll
    for (int v = 0; v < EV; v++) {
      const int e = tid + NT * v, r = e / CV, c = (e % CV) * 4, m = mp + r, n = n0 + c;
      if (m < M && n < N) {
        floatx4 es = {1.f, 1.f, 1.f, 1.f}, eb = {0.f, 0.f, 0.f, 0.f};
        if (o.emit.scale) {
          es = *(const floatx4*)(o.emit.scale + n);
          eb = *(const floatx4*)(o.emit.bias + n);
        }
        conv_store4<T>(o, m, n, *(const floatx4*)(Et + r * ELD + c), yres[v], rmv[v], es, eb, mkv[v]);
      }
    }
  }
}

// Tile configurations: narrow rows over all of a <= 192-wide N (1x1 convolutions, Winograd point GEMMs: the
// prologue runs once per element), 64x96 for 65..96 columns (the heads), 128x128 for wide GEMMs (transformer
// linears), 64x64 for the rest.
typedef Cfg<32, 192, 64, 1, 4, true> CfgNarrow;
typedef Cfg<128, 128, 64, 2, 2, true> CfgWide;
typedef Cfg<64, 64, 32, 2, 2> CfgSmall;
typedef Cfg<64, 96, 64, 2, 2, true> CfgHead;  // the heads' first convolutions: N = p1 + g1 + v1 channels <= 96

template <typename T, typename C, bool AF, bool PRO, int ACT>
static void gemm_launch(const GemmArgs& g, hipStream_t s) {
  if (g.qkv.dq && C::BN % g.qkv.dq)
    throw std::runtime_error("gemm: the q|k|v epilogue needs the column tile to hold whole heads");
  dim3 grid((g.N + C::BN - 1) / C::BN, (g.M + C::BM - 1) / C::BM, g.Z);
  gemm_kernel<T, C, AF, PRO, ACT><<<grid, C::WM * C::WN * 64, 0, s>>>(g);
}

template <typename T, bool AF, bool PRO, int ACT>
static void gemm_cfg(const GemmArgs& g, hipStream_t s) {
  const int bkh = 64, bk = sizeof(T) == 2 ? bkh : bkh / 2;
  if (g.N > 64 && g.N <= 96 && g.K % bk == 0) gemm_launch<T, CfgHead, AF, PRO, ACT>(g, s);
  else if (g.N > 128 && g.N <= 192 && g.K % bk == 0) gemm_launch<T, CfgNarrow, AF, PRO, ACT>(g, s);
  else if (g.N > 192 && g.N <= 384 && g.K % bk == 0 && AF) gemm_launch<T, CfgNarrow, AF, PRO, ACT>(g, s);
  else if (g.N > 128 && g.K % bk == 0 && (long)((g.M + 127) / 128) * ((g.N + 127) / 128) * g.Z >= 256)
    gemm_launch<T, CfgWide, AF, PRO, ACT>(g, s);
  else gemm_launch<T, CfgSmall, AF, PRO, ACT>(g, s);
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
