// Implicit-GEMM convolution for gfx950 on 16-bit operands: 1x1 and 3x3 "same" convolutions over NHWC
// activations as one MFMA GEMM per launch, out[m][o] = sum_{tap, i} x[m + shift(tap)][i] * w[tap][o][i], with
// m = n * 361 + y * 19 + x and shift(tap) = dy * 19 + dx (taps that leave the board contribute zero).
//
// At batch 32 and 192 channels a 3x3 convolution is about 7.7 GFLOP against 5 MB of operands: on CDNA4's matrix
// cores the direct contraction costs less than the Winograd transforms' extra traffic (F(2x2,3x3) writes and reads
// back four times the activation and streams 16/9 of the weights per output), and it rounds only the activation
// and the weights to 16 bits.
//
// A workgroup computes BM consecutive pixels x BN output channels. Per K stage (BK input channels) it stages in LDS
// the pixel rows [m0 - HALO, m0 + BM + HALO) (HALO = 20 covers every 3x3 neighbour) and the stage's weights of all
// taps (packed per N tile, [tile][tap][BN][icp], so a tile's weights are one contiguous block); each wave then
// runs TAPS x (BK / 32) MFMA steps over the staged data, reading the A fragment of tap t from
// the LDS row shifted by shift(t) and zeroing rows whose neighbour is off the board. The next stage's global loads
// are in flight in registers during the MFMAs. The epilogue goes through LDS so that every thread finishes four
// consecutive channels of one pixel with 16-byte loads and stores (conv_store4).
#include "kgx_device.h"

#include <cstring>
#include <vector>

namespace kgx {

template <int KS_, int BM_, int BN_, int BK_, int WM_, int WN_, int G_, int NBUF_, int MINW_ = 2,
          bool INTERLEAVE_ = false, bool SPLIT_ = false, bool WDMA_ = false>
struct IgCfg {
  // Weights straight into LDS (one 16-bit plane, one stage buffer for the pixel rows): each stage's weights go
  // from memory into one of two LDS buffers (buffer_load ... lds, 16 bytes per lane) while the previous stage's
  // MFMAs run, so only the pixel rows pass through registers and LDS store instructions. The weight rows are
  // BK = 64 channels (128 bytes) unpadded, their 16-byte chunks swizzled (chunk ^ (row / 2 % 8)), which keeps the
  // 16-row fragment reads conflict-free without the pad.
  static constexpr bool WDMA = WDMA_;
  // Split operands (1x1): the stage holds the high and the low plane of both operands, and each step takes
  // hi*hi + lo*hi + hi*lo (three MFMAs), a product of about 22 significant bits per operand.
  static constexpr bool SPLIT = SPLIT_;
  static constexpr int PL = SPLIT_ ? 2 : 1;     // operand planes per stage
  static constexpr int MINW = MINW_;            // waves per SIMD the register allocation must allow
  static constexpr bool INTERLEAVE = INTERLEAVE_;  // MFMA / LDS-read interleaving hints for the scheduler
  static constexpr int KS = KS_, TAPS = KS_ * KS_, HALO = KS_ == 3 ? POS + 1 : 0;
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int G = G_;                  // wave groups splitting the taps (partial sums added in LDS)
  static constexpr int NBUF = NBUF_;            // LDS stage buffers (2: the next stage is stored during the MFMAs)
  static constexpr int NT = WM * WN * 64 * G_;
  // 96-pixel tiles in pairs: both halves of a 192-pixel tile go to one XCD, as the 192-pixel convolutions around
  // them map it, so a layer still reads its input from the L2 its producer wrote.
  static constexpr bool PAIRS = BM_ == 96;
};

// XCD-aware tile order: workgroup g runs on XCD g % 8, so the ntl column tiles of one pixel tile are given the
// ids g, g + 8, ... of one XCD: they share its L2 for the pixel rows they all read, and their halves of the cache
// lines they write meet in the same L2. With 96-pixel tiles in pairs, both halves of a 192-pixel tile go to one
// XCD, as the 192-pixel convolutions around them map that tile. Workgroup g takes pixel tile mt and column tile
// nt; ids beyond the last pixel tile (the grid is rounded to 8) exit.
__host__ __device__ inline void igemm_tile_of(int g, int ntl, bool pairs, int& mt, int& nt) {
  const int slot = g >> 3, u = slot / ntl;
  nt = slot % ntl;
  mt = pairs ? 2 * ((u >> 1) * 8 + (g & 7)) + (u & 1) : u * 8 + (g & 7);
}

// Weights into LDS, one stage: wi instructions of 64 lanes fill the stage's wi * 8 weight rows of 128 bytes,
// instruction q of wave wv (nw waves) filling rows [8 (q nw + wv), + 8), lane i row i / 8 at stored chunk i % 8.
// Every wave issues the same number of instructions: one beyond the wi-th (q nw + wv >= wi) reloads the last 8
// rows into a spare area (dst_row8 = -1) that nothing reads, so that no load of the kernel sits under a branch.
__host__ __device__ inline void wdma_slot(int q, int wv, int lane, int nw, int wi, int& src_row, int& dst_row8) {
  const int ins = q * nw + wv;
  src_row = (ins < wi ? ins : wi - 1) * 8 + (lane >> 3);
  dst_row8 = ins < wi ? ins * 8 : -1;
}
// The stored 16-byte chunk of logical chunk c of weight row `row` (chunk ^ (row / 2 % 8)): conflict-free 16-row
// fragment reads of unpadded 128-byte rows. The swizzle is its own inverse, so a lane that stores chunk s loads the
// row's logical chunk wdma_chunk(row, s).
__host__ __device__ inline int wdma_chunk(int row, int c) { return c ^ ((row >> 1) & 7); }

// SC >= 0: the store case (store_flags, emitting mish if it emits), fixed by the launch so that the kernel holds only
// that store path; -1: every specialized case and the generic path, chosen from the arguments.
template <typename T, typename C, bool POOL, int SC = -1>
__global__ __launch_bounds__(C::NT, C::MINW) void igemm_kernel(const T* __restrict__ X, const T* __restrict__ Xlo,
                                                               int ldx, int IC, const T* __restrict__ W, int icp,
                                                               int OC, int M, ConvOut o) {
  constexpr int TAPS = C::TAPS, HALO = C::HALO, BM = C::BM, BN = C::BN, BK = C::BK, WM = C::WM, WN = C::WN;
  constexpr int NT = C::NT, G = C::G, PL = C::PL;
  static_assert(!C::SPLIT || C::KS == 1, "split operands: 1x1 only");
  // LDS row stride in elements: a 32-byte pad makes the 16-row fragment reads conflict-free (80 dwords apart rows
  // of a 16x16x32 fragment hit distinct banks; a 16-byte pad serialises them two-way on gfx950).
  constexpr int LDK = BK + 16;
  constexpr int KV = BK / 8;                  // 16-byte vectors per staged row
  constexpr int AR = BM + 2 * HALO;           // staged pixel rows (per operand plane)
  constexpr int TB = TAPS * BN;               // staged weight rows (per operand plane)
  constexpr int ZR = PL * AR;                 // the zero row
  constexpr int RP = NT / KV;                 // staged rows per pass of all threads
  constexpr int AV = (PL * AR + RP - 1) / RP, BV = (PL * TB + RP - 1) / RP;
  constexpr int WTM = BM / WM, WTN = BN / WN, MB = WTM / 16, NB = WTN / 16;
  static_assert(WTM % 16 == 0 && WTN % 16 == 0 && BK % 32 == 0 && NT % KV == 0, "bad tile");
  constexpr int STAGE = (PL * AR + 1 + PL * TB) * LDK * 2;  // bytes (A rows, a zero row, B rows)
  constexpr int EPI0 = C::G * BM * (BN + 4) * 4;      // bytes: one float tile per wave group
  // (then, with pooling partials, per wave, pooled channel and segment a sum and a maximum)
  constexpr int EPI = EPI0 + (POOL ? NT / 64 * 64 * 2 * 12 : 0);
  constexpr int NBUF = C::NBUF;
  constexpr int SE = STAGE / (int)sizeof(T);          // stage buffer size in elements
  static_assert(!C::WDMA || (NBUF == 1 && PL == 1 && BK == 64 && sizeof(T) == 2 && TB % 8 == 0 && BN % 16 == 0),
                "weights into LDS: one 16-bit plane of 128-byte rows, one pixel-row buffer");
  // Weights into LDS: two weight buffers of TB unpadded rows first (1 KB aligned, as each direct load fills one
  // KB), then the pixel rows and the zero row.
  constexpr int WSE = TB * BK;                          // weight buffer size in elements
  // (then, where the waves' direct loads do not divide the weight rows evenly, a spare KB for the surplus loads)
  constexpr int WSPARE = C::WDMA ? (2 * WSE * (int)sizeof(T) + (ZR + 1) * LDK * (int)sizeof(T) + 1023) / 1024 * 1024 : 0;
  constexpr int LDSB = C::WDMA ? WSPARE + ((TB / 8) % (NT / 64) ? 1024 : 0) : NBUF * STAGE;
  __shared__ __align__(1024) char smem[LDSB > EPI ? LDSB : EPI];
  T* Bw = (T*)smem;
  T* As = C::WDMA ? Bw + 2 * WSE : (T*)smem;
  T* Bs = As + (ZR + 1) * LDK;
  typedef u32x4 vec_t;
  typedef typename std::conditional<std::is_same<T, f16>::value, half8, bf16x8>::type frag_t;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave / (WM * WN), wl = wave - grp * (WM * WN);
  const int wm = wl / WN, wn = wl % WN;
  int mt, nt;
  igemm_tile_of(blockIdx.x, (OC + BN - 1) / BN, C::PAIRS, mt, nt);
  if (mt * BM >= M) {  // an idle workgroup still touches its share of the next launch's weights
    l2_touch_keep(l2_touch(o.pf, o.pf_bytes, threadIdx.x));
    return;
  }
  const int n0 = nt * BN, m0 = mt * BM;
  const int r16 = lane & 15, g4 = lane >> 4;

  // Staging: thread tid moves the 16-byte vector kv of rows r0, r0 + RP, r0 + 2 RP, ... of the stage's A rows
  // (pixels m0 - HALO + r; split: rows AR + r hold the low plane) and B rows (tap * BN + output channel of this N
  // tile, then the low plane, contiguous in the packed weights), so every address is a base plus a multiple of a
  // uniform stride.
  const int r0 = tid / KV, kv8 = (tid % KV) * 8;
  const T* wb = W + ((size_t)nt * PL * TB + r0) * icp + kv8;

  vec_t ra[AV], rb[BV];
  bool aok[AV];  // weights into LDS: whether pixel-row vector v holds real data (else it is stored as zeros)
  auto load = [&](int k0) {
    if constexpr (C::WDMA) {
      // Unconditional loads of clamped (in-range) rows, zeroed when stored where the row lies off the batch or
      // the channels beyond IC: with no branch around a load, the compiler's count of the loads issued after the
      // rows (the weights' direct loads) stays exact, so its wait before the row stores leaves those in flight.
#pragma unroll
      for (int v = 0; v < AV; v++) {
        const int r = r0 + v * RP;
        const int gr = m0 - HALO + r;
        aok[v] = gr >= 0 && gr < M && k0 + kv8 < IC;
        ra[v] = *(const vec_t*)(X + (size_t)min(max(gr, 0), M - 1) * ldx + (k0 + kv8 < IC ? k0 + kv8 : 0));
      }
      return;
    }
#pragma unroll
    for (int v = 0; v < AV; v++) {
      const int r = r0 + v * RP;
      const bool lo = C::SPLIT && r >= AR;
      const int gr = m0 - HALO + (lo ? r - AR : r);
      const bool ok = ((PL * AR) % RP == 0 || r < PL * AR) && gr >= 0 && gr < M && k0 + kv8 < IC;
      ra[v] = ok ? *(const vec_t*)((lo ? Xlo : X) + (size_t)gr * ldx + kv8 + k0) : vec_t{0, 0, 0, 0};
    }
    if constexpr (!C::WDMA) {
#pragma unroll
      for (int v = 0; v < BV; v++) {
        const bool ok = (PL * TB) % RP == 0 || r0 + v * RP < PL * TB;
        rb[v] = ok ? *(const vec_t*)(wb + (size_t)v * RP * icp + k0) : vec_t{0, 0, 0, 0};
      }
    }
  };
  auto store = [&](int buf) {
    T* ab = As + buf * SE + r0 * LDK + kv8;
    T* bb = Bs + buf * SE + r0 * LDK + kv8;
#pragma unroll
    for (int v = 0; v < AV; v++)
      if ((PL * AR) % RP == 0 || r0 + v * RP < PL * AR)
        *(vec_t*)(ab + v * RP * LDK) = !C::WDMA || aok[v] ? ra[v] : vec_t{0, 0, 0, 0};
    if constexpr (!C::WDMA) {
#pragma unroll
      for (int v = 0; v < BV; v++)
        if ((PL * TB) % RP == 0 || r0 + v * RP < PL * TB) *(vec_t*)(bb + v * RP * LDK) = rb[v];
    }
  };
  // Weights into LDS (wdma_slot): WQ direct loads per wave and stage, each lane loading the logical chunk that
  // its stored chunk holds. With no load under a branch, the compiler counts exactly how many direct loads follow
  // the pixel rows.
  constexpr int NW = NT / 64, WI = TB / 8, WQ = C::WDMA ? (WI + NW - 1) / NW : 1;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const T* wtile = W + (size_t)nt * PL * TB * icp;
  const int wbytes = TB * icp * (int)sizeof(T);
  T* const Wspare = (T*)(smem + WSPARE);
  int woff[WQ], wdst[WQ];
#pragma unroll
  for (int q = 0; q < WQ; q++) {
    int row;
    wdma_slot(q, wv, lane, NW, WI, row, wdst[q]);
    woff[q] = row * icp * (int)sizeof(T) + wdma_chunk(row, lane & 7) * 16;
  }
  auto issue_w = [&](int buf, int k0) {
    if constexpr (C::WDMA) {
#pragma unroll
      for (int q = 0; q < WQ; q++)
        lds_load16(wtile, wbytes, wdst[q] < 0 ? Wspare : Bw + buf * WSE + wdst[q] * BK, woff[q] + k0 * (int)sizeof(T));
    }
  };

  // The first stage's loads go out before the rest of the set-up (the tap masks, the epilogue's early loads), which
  // runs while they are in flight. Not in the 64-column 3x3: without partials, at 256 registers with its early
  // residual loads, it would spill; with partials it measured slower (its mask, staged in LDS before the main
  // loop, then waits behind the whole first stage).
  constexpr bool LOAD_FIRST = !(C::KS == 3 && C::BN == 64);
  // (Pixel rows before weights, as in every later stage: the compiler's wait before the row stores then leaves the
  // weights in flight on every path into the main loop.)
  if constexpr (LOAD_FIRST) {
    load(0);
    issue_w(0, 0);
  }

  // Tap validity of this lane's A rows: bit t of vmask[i] is set when row m's neighbour at tap t is on the board.
  unsigned vmask[MB];
#pragma unroll
  for (int i = 0; i < MB; i++) {
    const int m = m0 + wm * WTM + i * 16 + r16;
    unsigned bits = 0;
    if (m < M) {
      const int p = m % HW, y = p / POS, x = p - y * POS;
#pragma unroll
      for (int t = 0; t < TAPS; t++) {
        const int dy = C::KS == 3 ? t / 3 - 1 : 0, dx = C::KS == 3 ? t % 3 - 1 : 0;
        if ((unsigned)(y + dy) < (unsigned)POS && (unsigned)(x + dx) < (unsigned)POS) bits |= 1u << t;
      }
    }
    vmask[i] = bits;
  }

  floatx4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // The MFMA steps of one group over the staged stage: its share of the (tap, 32-channel slice) pairs, with the
  // fragments of the next step read from LDS while the current step's MFMAs run.
  // Fragment reads of the swizzled weight rows: fragment rows start at multiples of 16, so a row's swizzle is that
  // of row r16, and lane group g4's chunk of K offset kk is wdma_chunk(r16, kk / 8 ^ g4).
  auto mma = [&](auto gc, int sb, int wbuf) {
    constexpr int g = decltype(gc)::value;
    constexpr int KK = BK / 32, ST = TAPS * KK, S0 = g * ST / G, S = (g + 1) * ST / G - S0;
    frag_t a[2][MB], b[2][NB];
    frag_t al[C::SPLIT ? 2 : 1][MB], bl[C::SPLIT ? 2 : 1][NB];  // low planes (split)
    auto fetch = [&](int s, int fb) {
      const int t = (S0 + s) / KK, kk = ((S0 + s) % KK) * 32;
      const int shift = C::KS == 3 ? (t / 3 - 1) * POS + (t % 3 - 1) : 0;
      const T* bs = C::WDMA ? Bw + wbuf * WSE + (t * BN + wn * WTN + r16) * BK + wdma_chunk(r16, (kk / 8) ^ g4) * 8
                            : Bs + sb * SE + (t * BN + wn * WTN + r16) * LDK + g4 * 8 + kk;
#pragma unroll
      for (int i = 0; i < MB; i++) {
        // Rows whose neighbour is off the board read the zero row, so no loaded value needs masking.
        const bool on = (vmask[i] >> t) & 1;
        const int row = on ? wm * WTM + i * 16 + r16 + HALO + shift : ZR;
        a[fb][i] = *(const frag_t*)(As + sb * SE + row * LDK + g4 * 8 + kk);
        if constexpr (C::SPLIT) al[fb][i] = *(const frag_t*)(As + sb * SE + (on ? row + AR : ZR) * LDK + g4 * 8 + kk);
      }
#pragma unroll
      for (int j = 0; j < NB; j++) {
        b[fb][j] = *(const frag_t*)(bs + j * 16 * (C::WDMA ? BK : LDK));
        if constexpr (C::SPLIT) bl[fb][j] = *(const frag_t*)(bs + (TB + j * 16) * LDK);
      }
    };
    auto mfma = [&](const frag_t& x, const frag_t& y, floatx4 c) {
      if constexpr (std::is_same<T, f16>::value) return __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c, 0, 0, 0);
      else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, c, 0, 0, 0);
    };
    fetch(0, 0);
#pragma unroll
    for (int s = 0; s < S; s++) {
      if (s + 1 < S) fetch(s + 1, (s + 1) & 1);
      // Keep the order: all of the next step's LDS reads are issued before this step's MFMAs (the scheduler
      // would otherwise move each read next to its first use and expose the LDS latency on every step).
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (C::SPLIT) {
        // The two correction terms first (independent accumulators back to back), then the main product.
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < NB; j++) acc[i][j] = mfma(al[s & 1][i], b[s & 1][j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < NB; j++) acc[i][j] = mfma(a[s & 1][i], bl[s & 1][j], acc[i][j]);
      }
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = mfma(a[s & 1][i], b[s & 1][j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (C::INTERLEAVE) {
        // Scheduling hint: alternate this step's MFMAs with the next step's LDS fragment reads.
#pragma unroll
        for (int k = 0; k < MB * NB; k++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          if (s + 1 < S && k < MB + NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
        }
      }
    }
  };

  auto compute = [&](int buf, int wbuf = 0) {
    if constexpr (G == 1) {
      mma(std::integral_constant<int, 0>{}, buf, wbuf);
    } else {
      if (grp == 0) mma(std::integral_constant<int, 0>{}, buf, wbuf);
      else mma(std::integral_constant<int, G - 1>{}, buf, wbuf);
    }
  };
  // Epilogue mapping: thread tid finishes the four channels 4 * (tid % G4) of rows tid / G4 + e * RPE, so its
  // emit scale and bias are loaded once. The 3x3 kernel reads the residual values before the main loop so that the
  // reads overlap it (the variant with pooling partials after), and on 48-column tiles also the masks and emit
  // parameters (0.4-1 us less per conv than after the loop); the split 192-pixel 1x1 reads the residual early too;
  // the wider 3x3 tiles and the other 1x1 kernels read the rest after (read early they spill: the 1x1 is held to
  // 128 registers for two workgroups per CU).
  constexpr int G4 = BN / 4, RPE = NT / G4, EV = (BM + RPE - 1) / RPE;
  constexpr bool YEARLY = (C::KS == 3 && !POOL) || (C::SPLIT && C::BK == 64 && !C::PAIRS);
  constexpr bool SEARLY = YEARLY && C::BN <= 48;  // wider column tiles would spill with these registers live
  const int ec4 = tid % G4, er0 = tid / G4, en = n0 + 4 * ec4;
  const bool eon = er0 < RPE && en < OC;
  // Loads use clamped pixel and channel indices (always in range, no branches, so they issue back to back);
  // the stores below skip what lies outside the tile.
  const int enc = min(en, OC - 4);
  auto epix = [&](int e) { return min(m0 + min(er0 + e * RPE, BM - 1), M - 1); };
  const bool yacc = o.y && o.accumulate;
  // Each input is loaded under one uniform branch and left undefined otherwise (no per-element control flow,
  // so the loads issue back to back).
  floatx4 yres[EV];
  auto load_y = [&]() {
    if (yacc) {
#pragma unroll
      for (int e = 0; e < EV; e++) yres[e] = *(const floatx4*)(o.y + (size_t)epix(e) * o.ldy + enc);
    }
  };
  float rmv[EV], mkv[EV];
  floatx4 es, eb;
  auto load_side = [&]() {
    if (o.emit.scale) {
      es = *(const floatx4*)(o.emit.scale + enc);
      eb = *(const floatx4*)(o.emit.bias + enc);
#pragma unroll
      for (int e = 0; e < EV; e++) mkv[e] = o.emit.mask[epix(e)];
    }
    if (o.rowmask) {
#pragma unroll
      for (int e = 0; e < EV; e++) rmv[e] = o.rowmask[epix(e)];
    }
  };
  if constexpr (YEARLY) load_y();
  if constexpr (SEARLY) load_side();
  // Board pooling partials (PoolPart): the tile's last CT = BN - pp.rpt columns are pooled channels, summed and
  // maxed per segment of the tile (the batch row of its first pixel, and the next one) and not stored; the regular
  // columns before them go to y column ycol. The pooling pass has a mapping of its own: thread tid takes pooled
  // channel pch = tid % CT of rows prow0 + j * pstep (CT a power of two from 4 to 64, so that the lanes holding
  // one channel are CT apart in every wave). Its scale and bias, and the tile's board mask (into LDS), are read
  // here, before the main loop, so that the pass waits for no memory.
  const PoolPart& pp = o.pool;
  const int ycol = POOL ? nt * pp.rpt + 4 * ec4 : en;
  const bool pcol = POOL && 4 * ec4 >= pp.rpt;  // this thread's store columns are pooled
  const int lct = POOL ? __builtin_ctz(BN - pp.rpt) : 0, CT = 1 << lct;
  const int pch = tid & (CT - 1), prow0 = tid >> lct, pstep = NT >> lct;
  __shared__ float pms[POOL ? BM : 1];
  float psc, pbi, pmv;
  if constexpr (POOL) {
    static_assert(NT >= BM, "pooling partials: a thread per pixel row stages the mask");
    psc = pp.scale[nt * CT + pch];
    pbi = pp.bias[nt * CT + pch];
    pmv = pp.mask[min(m0 + min(tid, BM - 1), M - 1)];
  }

  // The zero row of every stage buffer (never written by the stage stores).
  for (int e = tid; e < NBUF * KV; e += NT) *(vec_t*)(As + (e / KV) * SE + ZR * LDK + (e % KV) * 8) = vec_t{0, 0, 0, 0};
  const int nk = icp / BK;
  if constexpr (!LOAD_FIRST) {
    load(0);
    issue_w(0, 0);
  }
  if constexpr (POOL) {
    if (tid < BM) pms[tid] = pmv;  // ordered before the pass by the main loop's barriers
  }
  if constexpr (C::WDMA) {
    // Pixel rows: store, barrier, next loads in flight during the MFMAs, barrier. Weights: stage kt + 1 streams
    // into the other weight buffer while stage kt's MFMAs run. The pixel rows are ordinary loads issued before the
    // stage's direct weight loads, so the wait the compiler places before the row stores (it counts both kinds)
    // leaves the weights in flight while the rows are stored. The compiler does not order LDS reads after direct
    // loads into LDS, so each wave waits for all of its loads before the barrier that publishes the stage.
    for (int kt = 0; kt < nk; kt++) {
      store(0);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (kt + 1 < nk) {
        load((kt + 1) * BK);
        issue_w((kt + 1) & 1, (kt + 1) * BK);
      }
      compute(0, kt & 1);
      // Every wave is done reading this stage from LDS before the next row stores and weight loads overwrite it.
      // The barrier waits for this wave's LDS reads only: a fence (__syncthreads(), or one scoped to LDS) would
      // also wait for the next stage's loads in flight, the direct ones counting as LDS writes. The compiler
      // moves no memory access across the two clobbers, nor the clobbers across the barrier.
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("" ::: "memory");
    }
  } else if constexpr (NBUF == 1) {
    // One stage buffer: store, barrier, next loads in flight during the MFMAs, barrier.
    for (int kt = 0; kt < nk; kt++) {
      store(0);
      __syncthreads();
      if (kt + 1 < nk) load((kt + 1) * BK);
      compute(0);
      __syncthreads();
    }
  } else {
    // Two stage buffers: the next stage's loads are issued before and stored after the current MFMAs; one barrier.
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
      if (kt + 1 < nk) load((kt + 1) * BK);
      compute(kt & 1);
      if (kt + 1 < nk) store((kt + 1) & 1);
      __syncthreads();
    }
  }

  // Accumulators to LDS, one float [BM][BN + 4] tile per wave group, summed per output vector: element (i, j, r)
  // is row wm*WTM + i*16 + 4*(lane/16) + r, column wn*WTN + j*16 + lane%16.
  constexpr int LDC = BN + 4;
  float* Cs = (float*)smem;
  float* Cg = Cs + grp * BM * LDC;
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) Cg[(wm * WTM + i * 16 + 4 * g4 + r) * LDC + wn * WTN + j * 16 + r16] = acc[i][j][r];
  __syncthreads();
  // The other epilogue inputs, loaded after the accumulator exchange and before the first store.
  if constexpr (!YEARLY) load_y();
  if constexpr (!SEARLY) load_side();

  // The stores, in one copy per emission activation, and for mish per set of outputs that the networks' convs
  // ask for (store_flags): the epilogue runs once per workgroup from a cold instruction cache, where one
  // contiguous path is faster than a branch per value.
  auto store_rows = [&](auto act_c, auto fl_c) {
#pragma unroll
    for (int e = 0; e < EV; e++) {
      const int row = er0 + e * RPE, m = m0 + row;
      if (eon && !pcol && row < BM && m < M) {
        floatx4 sum = *(const floatx4*)(Cs + row * LDC + 4 * ec4);
#pragma unroll
        for (int q = 1; q < G; q++) sum += *(const floatx4*)(Cs + q * BM * LDC + row * LDC + 4 * ec4);
        conv_store4<T, decltype(act_c)::value, decltype(fl_c)::value>(o, m, ycol, sum, yres[e], rmv[e], es, eb,
                                                                       mkv[e]);
      }
    }
  };
  typedef std::integral_constant<int, ACT_MISH> Mish;
  typedef std::integral_constant<int, -1> AnyFlags;
  // (Not for the 64-column 3x3 without partials: at 256 registers with its early residual loads, it spills.)
  constexpr bool SPEC = !(C::KS == 3 && C::BN == 64 && !POOL);
  const int sfl = store_flags(o);
  const int scase = SC >= 0 ? SC : !SPEC ? -1 : !(sfl & SF_EMIT) ? sfl : o.emit.act == ACT_MISH ? sfl : -1;
  // The next launch's weights into this XCD's L2 while the epilogue runs. Issued after every load that the stores
  // wait for, and only where the stores load nothing more (the specialized cases other than the column bias's),
  // since a wait for a later load would include it.
  bool quiet = false;
  switch (scase) {
    case SF_Y: case SF_EMIT: case SF_Y | SF_EMIT: case SF_Y | SF_ACC | SF_EMIT: case SF_Y | SF_ACC | SF_YDEAD | SF_EMIT:
    case SF_Y | SF_ACC | SF_EMIT | SF_LO: case SF_Y | SF_ACC | SF_YDEAD | SF_EMIT | SF_LO: quiet = true; break;
    default: break;
  }
  const int pfv = l2_touch(o.pf, quiet ? o.pf_bytes : 0, tid);
  // With pooling partials the regular columns are a plain float output (the host admits no other), or nothing when
  // the stream is dead: only that path is built, which keeps the kernel's code to what it runs.
  if constexpr (POOL) {
    if (scase == SF_Y) store_rows(std::integral_constant<int, ACT_ID>{}, std::integral_constant<int, SF_Y>{});
  } else if constexpr (SC >= 0) {
    store_rows(std::integral_constant<int, (SC & SF_EMIT) ? ACT_MISH : ACT_ID>{}, std::integral_constant<int, SC>{});
  } else switch (scase) {
    // a global-pooling block's first conv (pooling partials); a block's first conv; a nested block's entry 1x1;
    // a block's last conv, its stream's last, into a split 1x1
    case SF_Y: store_rows(std::integral_constant<int, ACT_ID>{}, std::integral_constant<int, SF_Y>{}); break;
    case SF_EMIT: store_rows(Mish{}, std::integral_constant<int, SF_EMIT>{}); break;
    case SF_Y | SF_EMIT: store_rows(Mish{}, std::integral_constant<int, SF_Y | SF_EMIT>{}); break;
    case SF_Y | SF_ACC | SF_EMIT: store_rows(Mish{}, std::integral_constant<int, SF_Y | SF_ACC | SF_EMIT>{}); break;
    case SF_Y | SF_ACC | SF_YDEAD | SF_EMIT:
      store_rows(Mish{}, std::integral_constant<int, SF_Y | SF_ACC | SF_YDEAD | SF_EMIT>{});
      break;
    case SF_Y | SF_ACC | SF_EMIT | SF_LO:
      store_rows(Mish{}, std::integral_constant<int, SF_Y | SF_ACC | SF_EMIT | SF_LO>{});
      break;
    case SF_Y | SF_ACC | SF_YDEAD | SF_EMIT | SF_LO:  // the trunk's last conv into the split head 1x1
      store_rows(Mish{}, std::integral_constant<int, SF_Y | SF_ACC | SF_YDEAD | SF_EMIT | SF_LO>{});
      break;
    case SF_COLBIAS | SF_Y | SF_EMIT | SF_LO:  // the stem into a nested block's entry 1x1
      store_rows(Mish{}, std::integral_constant<int, SF_COLBIAS | SF_Y | SF_EMIT | SF_LO>{});
      break;
    default:
      switch (o.emit.act) {
        case ACT_RELU: store_rows(std::integral_constant<int, ACT_RELU>{}, AnyFlags{}); break;
        case ACT_MISH: store_rows(Mish{}, AnyFlags{}); break;
        case ACT_SILU: store_rows(std::integral_constant<int, ACT_SILU>{}, AnyFlags{}); break;
        default: store_rows(std::integral_constant<int, ACT_ID>{}, AnyFlags{}); break;
      }
  }

  if constexpr (POOL) {
    // The pooling pass, after the stores (they drain meanwhile: its barrier waits for LDS only). Fixed-point sums as two 32-bit
    // parts: round(x * 2^24) = hi * 2^24 + lo with hi = floor(x) and lo = round((x - hi) * 2^24) in [0, 2^24],
    // exact per value, and summed exactly over a tile's 192 pixels for |x| < 2^23 (clamped there): hi as int,
    // lo as unsigned (at most 192 * 2^24 < 2^32). Rows from r1 on belong to the next batch row (segment 1).
    const int b0 = m0 / HW, r1 = (b0 + 1) * HW - m0, rows = min(BM, M - m0), pcl = pp.rpt + pch;
    int h0 = 0, h1 = 0;
    unsigned l0 = 0, l1 = 0;
    float x0 = -FLT_MAX, x1 = -FLT_MAX;
    // A rolled loop per activation: the pass runs once per workgroup, from a cold instruction cache.
    auto pool_rows = [&](auto act_c) {
      constexpr int A = decltype(act_c)::value;
#pragma unroll 1
      for (int row = prow0; row < rows; row += pstep) {
        float a = Cs[row * LDC + pcl];
#pragma unroll
        for (int q = 1; q < G; q++) a += Cs[q * BM * LDC + row * LDC + pcl];
        const float mk = pms[row], x = act_f<A>(a * psc + pbi) * mk, pen = mk * 1e4f - 1e4f;
        const float xc = fminf(fmaxf(x, -8388607.f), 8388607.f), h = floorf(xc);
        const int qh = (int)h;
        const unsigned ql = (unsigned)rintf((xc - h) * kPoolFix);
        if (row >= r1) {
          h1 += qh; l1 += ql; x1 = fmaxf(x1, x + pen);
        } else {
          h0 += qh; l0 += ql; x0 = fmaxf(x0, x + pen);
        }
      }
    };
    switch (pp.act) {
      case ACT_RELU: pool_rows(std::integral_constant<int, ACT_RELU>{}); break;
      case ACT_MISH: pool_rows(std::integral_constant<int, ACT_MISH>{}); break;
      case ACT_SILU: pool_rows(std::integral_constant<int, ACT_SILU>{}); break;
      default: pool_rows(std::integral_constant<int, ACT_ID>{}); break;
    }
    // Lanes pch, pch + CT, ... of a wave hold the same channel: summed by row rotations within 16-lane rows (DPP,
    // for CT 4 and 8) and lane swaps across rows (v_permlane16_swap / v_permlane32_swap in inline assembly: the
    // builtins fold both results into one when both operands hold the same value), so that lane pch holds the
    // wave's total. The waves' totals then meet in LDS after the accumulator tiles and are reduced in wave order;
    // segment 1 is written only when the tile reaches into the next batch row.
    auto red = [&](auto v, auto op) {
      typedef decltype(v) V;
      auto rot = [&](V u, auto ctl) -> V {
        return __builtin_bit_cast(V, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, u), decltype(ctl)::value,
                                                                 0xf, 0xf, false));
      };
      if (CT <= 4) v = op(v, rot(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
      if (CT <= 8) v = op(v, rot(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
      if (CT <= 16) {
        V a = v, b = v;
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        v = op(a, b);
      }
      if (CT <= 32) {
        V a = v, b = v;
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        v = op(a, b);
      }
      return v;
    };
    auto add_i = [](int a, int b) { return a + b; };
    auto add_u = [](unsigned a, unsigned b) { return a + b; };
    auto max_f = [](float a, float b) { return fmaxf(a, b); };
    h0 = red(h0, add_i); h1 = red(h1, add_i);
    l0 = red(l0, add_u); l1 = red(l1, add_u);
    x0 = red(x0, max_f); x1 = red(x1, max_f);
    constexpr int NW = NT / 64;
    long long* RS = (long long*)(smem + EPI0);  // [wave][channel][segment]
    float* RX = (float*)(RS + NW * 64 * 2);
    if (lane < CT) {
      const int at = ((tid >> 6) * 64 + lane) * 2;
      RS[at] = (long long)h0 * (1 << 24) + (long long)l0;
      RS[at + 1] = (long long)h1 * (1 << 24) + (long long)l1;
      RX[at] = x0;
      RX[at + 1] = x1;
    }
    __syncthreads();
    const bool has1 = r1 < rows;
    if (tid < 4 * CT) {
      const int ch = tid & (CT - 1), seg = (tid >> lct) & 1, isMax = tid >> (lct + 1);
      if (seg == 0 || has1) {
        const size_t at = (size_t)(mt * 2 + seg) * pp.C + nt * CT + ch;
        if (isMax) {
          float v = -FLT_MAX;
#pragma unroll
          for (int w = 0; w < NW; w++) v = fmaxf(v, RX[(w * 64 + ch) * 2 + seg]);
          pp.pmax[at] = v;
        } else {
          long long v = 0;
#pragma unroll
          for (int w = 0; w < NW; w++) v += RS[(w * 64 + ch) * 2 + seg];
          pp.psum[at] = v;
        }
      }
    }
  }
  l2_touch_keep(pfv);
}

// Configurations (measured at batch 32, 192 channels): 3x3 with 192 pixels x 48 channels per workgroup (a
// quarter of the weights per workgroup: weight staging is what bounds this kernel), 64 channels per stage and two
// wave groups of 4x1 waves (48x48 each) splitting the taps; 1x1 on the same 192-pixel tiles with two stage
// buffers. Equal pixel tiles give every convolution the same tile -> XCD mapping, so a layer reads the
// activations its producer wrote from the same XCD's L2. The 1x1 kernel keeps two workgroups per CU (four waves
// per SIMD, at most 128 registers): its 384-channel outputs are 512 workgroups.
typedef IgCfg<3, 192, 48, 64, 4, 1, 2, 1, 2, false, false, true> Ig3;
typedef IgCfg<1, 192, 48, 64, 4, 1, 2, 2, 4> Ig1;
// Wider output tiles keep a 3x3 convolution with more than 192 output channels at four column tiles (one wave
// of workgroups on 256 CUs at batch 32): 64 channels for up to 256 (a global-pooling block's first conv), 96 for
// up to 384 (the stem), the latter on 32-channel stages with all eight waves on every tap (its weights for all
// taps of 96 channels would not fit LDS at 64 channels per stage).
typedef IgCfg<3, 192, 64, 64, 4, 1, 2, 1> Ig3n64;
typedef IgCfg<3, 192, 96, 32, 4, 2, 1, 1> Ig3n96;
// A 1x1 over a multiple of 128 input channels into at most 192 outputs (a nested-bottleneck block's first conv,
// one wave of workgroups at batch 32) takes 128 channels per stage, one stage buffer: half the stages, 10.2-10.7
// against 11.3-12.0 us at 384 -> 192.
typedef IgCfg<1, 192, 48, 128, 4, 1, 2, 1, 2> Ig1k128;
// Split-operand 1x1 (float-accurate): the same tiles with both operand planes staged, one workgroup per CU
// (138.5 KB of LDS at 128 channels per stage; 154 KB for two 64-channel stage buffers).
typedef IgCfg<1, 192, 48, 128, 4, 1, 2, 1, 2, false, true> Ig1k128s;
// Any other split 1x1 (each nested block's last conv, 192 -> 384) on 96-pixel x 96-channel tiles in XCD pairs, two
// workgroups per CU so that one's epilogue (the float trunk read and written, the activation emitted in two
// planes) overlaps the other's loads and MFMAs: 16.5 -> 15.9-16.3 us against 192x96 tiles (+0.3-0.9 % end to
// end, two boxes). Measured beside it: the same for the 384 -> 192 entry 1x1 (96x48 tiles, 64-channel stages):
// 12.9 -> 12.5 us but no end-to-end gain.
typedef IgCfg<1, 96, 96, 64, 2, 2, 1, 1, 2, false, true> Ig1sh;

enum { IG3_48, IG3_64, IG3_96, IG1_48, IG1_128, IG1_48S, IG1_128S };
static int igemm_kind(int ks, int ic, int oc, bool split) {
  if (ks == 1 && split) return ic % Ig1k128s::BK == 0 && oc <= 4 * Ig1k128s::BN ? IG1_128S : IG1_48S;
  if (ks == 1) return ic % Ig1k128::BK == 0 && oc <= 4 * Ig1k128::BN ? IG1_128 : IG1_48;
  if (oc <= 4 * Ig3::BN) return IG3_48;
  if (oc <= 4 * Ig3n64::BN) return IG3_64;
  return IG3_96;
}
static void igemm_tile(int kind, int& bn, int& bk) {
  switch (kind) {
    case IG3_48: bn = Ig3::BN; bk = Ig3::BK; break;
    case IG3_64: bn = Ig3n64::BN; bk = Ig3n64::BK; break;
    case IG3_96: bn = Ig3n96::BN; bk = Ig3n96::BK; break;
    case IG1_128: bn = Ig1k128::BN; bk = Ig1k128::BK; break;
    case IG1_128S: bn = Ig1k128s::BN; bk = Ig1k128s::BK; break;
    case IG1_48S: bn = Ig1sh::BN; bk = Ig1sh::BK; break;
    default: bn = Ig1::BN; bk = Ig1::BK; break;
  }
}

template <typename T, typename C>
static void igemm_launch(const void* x, const void* xlo, int ldx, int IC, const void* w, int icp, int OC,
                         const ConvOut& o, int M, hipStream_t s) {
  if (icp % C::BK != 0) throw std::runtime_error("conv_igemm: padded input channels must be a multiple of the stage");
  const int mtiles = (M + C::BM - 1) / C::BM, ntiles = (OC + C::BN - 1) / C::BN;
  // Pairs: ceil(pairs / 8) pairs per XCD, two tiles each.
  dim3 grid(C::PAIRS ? 8 * ((mtiles + 15) / 16) * 2 * ntiles : round_up(mtiles, 8) * ntiles);
  if constexpr (C::KS == 3 && 64 % (C::BN / 4) == 0) {
    if (o.pool.psum) {
      launch_k(igemm_kernel<T, C, true>, grid, C::NT, 0, s, (const T*)x, (const T*)xlo, ldx, IC, (const T*)w, icp, OC,
               M, o);
      return;
    }
  }
  if (o.pool.psum) throw std::runtime_error("conv_igemm: no pooling partials for this convolution's tile");
  auto go = [&](auto kernel) {
    launch_k(kernel, grid, C::NT, 0, s, (const T*)x, (const T*)xlo, ldx, IC, (const T*)w, icp, OC, M, o);
  };
  if constexpr (C::WDMA) {
    // The 48-column 3x3 (most of a residual trunk's launches): one kernel per store case that the networks' convs
    // ask for, each holding only its own store path. Measured on the pooled 3x3, whose kernel dropped from 9.4k to
    // 2.2k instructions that way, the smaller kernel ran 0.6 us faster with the same executed path.
    const int sfl = store_flags(o);
    switch ((sfl & SF_EMIT) && o.emit.act != ACT_MISH ? -1 : sfl) {
      case SF_EMIT: go(igemm_kernel<T, C, false, SF_EMIT>); return;
      case SF_Y: go(igemm_kernel<T, C, false, SF_Y>); return;
      case SF_Y | SF_EMIT: go(igemm_kernel<T, C, false, SF_Y | SF_EMIT>); return;
      case SF_Y | SF_ACC | SF_EMIT: go(igemm_kernel<T, C, false, SF_Y | SF_ACC | SF_EMIT>); return;
      case SF_Y | SF_ACC | SF_YDEAD | SF_EMIT: go(igemm_kernel<T, C, false, SF_Y | SF_ACC | SF_YDEAD | SF_EMIT>); return;
      case SF_Y | SF_ACC | SF_EMIT | SF_LO: go(igemm_kernel<T, C, false, SF_Y | SF_ACC | SF_EMIT | SF_LO>); return;
      case SF_Y | SF_ACC | SF_YDEAD | SF_EMIT | SF_LO:
        go(igemm_kernel<T, C, false, SF_Y | SF_ACC | SF_YDEAD | SF_EMIT | SF_LO>);
        return;
      default: break;
    }
  }
  go(igemm_kernel<T, C, false>);
}

template <typename T>
static void igemm_dispatch(int kind, const void* x, const void* xlo, int ldx, int IC, const void* w, int icp, int OC,
                           const ConvOut& o, int M, hipStream_t s) {
  switch (kind) {
    case IG3_48: igemm_launch<T, Ig3>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
    case IG3_64: igemm_launch<T, Ig3n64>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
    case IG3_96: igemm_launch<T, Ig3n96>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
    case IG1_128: igemm_launch<T, Ig1k128>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
    case IG1_128S: igemm_launch<T, Ig1k128s>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
    case IG1_48S: igemm_launch<T, Ig1sh>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
    default: igemm_launch<T, Ig1>(x, xlo, ldx, IC, w, icp, OC, o, M, s); break;
  }
}

thread_local LaunchTiming g_launch_timing;

template <typename C>
static IgemmGeometry igemm_geometry_of(int OC, int M) {
  IgemmGeometry gm;
  const int mtiles = (M + C::BM - 1) / C::BM, ntiles = (OC + C::BN - 1) / C::BN;
  gm.grid = C::PAIRS ? 8 * ((mtiles + 15) / 16) * 2 * ntiles : round_up(mtiles, 8) * ntiles;  // as igemm_launch
  gm.threads = C::NT;
  gm.tile_rows = C::BM;
  gm.tile_cols = C::BN;
  gm.stage_channels = C::BK;
  gm.col_tiles = ntiles;
  gm.pixel_tiles = mtiles;
  gm.pairs = C::PAIRS;
  gm.weights_direct = C::WDMA;
  gm.weight_rows = C::TAPS * C::BN;
  gm.waves = C::NT / 64;
  gm.direct_instructions = C::WDMA ? C::TAPS * C::BN / 8 : 0;
  gm.direct_per_wave = C::WDMA ? (gm.direct_instructions + gm.waves - 1) / gm.waves : 0;
  return gm;
}

IgemmGeometry conv_igemm_geometry(int ks, int ic, int oc, bool split, int M) {
  switch (igemm_kind(ks, ic, oc, split)) {
    case IG3_48: return igemm_geometry_of<Ig3>(oc, M);
    case IG3_64: return igemm_geometry_of<Ig3n64>(oc, M);
    case IG3_96: return igemm_geometry_of<Ig3n96>(oc, M);
    case IG1_128: return igemm_geometry_of<Ig1k128>(oc, M);
    case IG1_128S: return igemm_geometry_of<Ig1k128s>(oc, M);
    case IG1_48S: return igemm_geometry_of<Ig1sh>(oc, M);
    default: return igemm_geometry_of<Ig1>(oc, M);
  }
}

void conv_igemm_tile_of(const IgemmGeometry& gm, int g, int& mt, int& nt) {
  igemm_tile_of(g, gm.col_tiles, gm.pairs, mt, nt);
  if (mt >= gm.pixel_tiles) mt = nt = -1;
}

void conv_igemm_weight_load(const IgemmGeometry& gm, int q, int wave, int lane, int& src_row, int& src_chunk,
                            int& dst_row, int& dst_chunk) {
  int row8;
  wdma_slot(q, wave, lane, gm.waves, gm.direct_instructions, src_row, row8);
  src_chunk = wdma_chunk(src_row, lane & 7);
  dst_row = row8 < 0 ? -1 : row8 + (lane >> 3);
  dst_chunk = lane & 7;
}

int conv_igemm_weight_chunk(int row, int chunk) { return wdma_chunk(row, chunk); }

const char* conv_igemm_class(int ks, int ic, int oc, bool split) {
  switch (igemm_kind(ks, ic, oc, split)) {
    case IG3_48: return "conv3x3";
    case IG3_64: return "conv3x3_n64";
    case IG3_96: return "conv3x3_n96";
    case IG1_128: return "conv1x1_k128";
    case IG1_128S: return "conv1x1_split_k128";
    case IG1_48S: return "conv1x1_split_n96";
    default: return "conv1x1";
  }
}

int conv_igemm_pool_cols(int ks, int ic, int oc) {
  // The 3x3 tiles of 64 columns (16 channel groups: the lane swaps of the partials' reduction), 192 pixels each.
  return igemm_kind(ks, ic, oc, false) == IG3_64 ? Ig3n64::BN : 0;
}

int conv_igemm_tile_rows(int ks, int ic, int oc, bool split) {
  switch (igemm_kind(ks, ic, oc, split)) {
    case IG3_48: return Ig3::BM;
    case IG3_64: return Ig3n64::BM;
    case IG3_96: return Ig3n96::BM;
    case IG1_128: return Ig1k128::BM;
    case IG1_128S: return Ig1k128s::BM;
    case IG1_48S: return Ig1sh::BM;
    default: return Ig1::BM;
  }
}

int conv_igemm_icp(int ks, int ic, int oc, bool split) {
  int bn, bk;
  igemm_tile(igemm_kind(ks, ic, oc, split), bn, bk);
  return round_up(ic, bk);
}

float conv_round_operand(float v, int prec) {
  if (prec == PREC_BF16) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return v;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
  }
  return (float)(_Float16)v;
}

// w [oc][ic][ks][ks] -> [oc tile][plane][tap][BN][icp], zero padding beyond oc and ic (BN and icp of the
// configuration launch_conv_igemm picks for these channel counts); one plane, or with `split` the high plane and
// the low plane w - round(w).
void conv_igemm_pack_weights(int ks, const float* w, int oc, int ic, std::vector<float>& out, bool split, int prec) {
  if (split && ks != 1) throw std::runtime_error("conv_igemm: split operands for 1x1 convolutions only");
  int bn, bk;
  igemm_tile(igemm_kind(ks, ic, oc, split), bn, bk);
  const int taps = ks * ks, icp = round_up(ic, bk), pl = split ? 2 : 1;
  const int tiles = (oc + bn - 1) / bn;
  out.assign((size_t)tiles * pl * taps * bn * icp, 0.f);
  for (int o = 0; o < oc; o++)
    for (int t = 0; t < taps; t++)
      for (int i = 0; i < ic; i++) {
        const float v = w[((size_t)o * ic + i) * taps + t];
        const size_t hi = ((((size_t)(o / bn) * pl) * taps + t) * bn + o % bn) * icp + i;
        out[hi] = v;
        if (split) out[hi + (size_t)taps * bn * icp] = v - conv_round_operand(v, prec);
      }
}

void launch_conv_igemm(int prec, int ks, const void* x, int ldx, int IC, const void* w, int icp, int OC,
                       const ConvOut& o, int B, hipStream_t s, const void* x_lo) {
  if (prec != PREC_F16 && prec != PREC_BF16) throw std::runtime_error("conv_igemm: 16-bit operands only");
  if (ks != 1 && ks != 3) throw std::runtime_error("conv_igemm: 1x1 or 3x3 kernels only");
  if (x_lo && ks != 1) throw std::runtime_error("conv_igemm: split operands for 1x1 convolutions only");
  const bool split = x_lo != nullptr;
  if (IC % 8 != 0 || ldx % 8 != 0 || OC % 4 != 0 || icp != conv_igemm_icp(ks, IC, OC, split))
    throw std::runtime_error("conv_igemm: channel counts must be multiples of 8 (inputs) and 4 (outputs)");
  if ((o.y && o.ldy % 4) || (o.yt && o.ldyt % 4) || (o.colbias && o.ld_colbias % 4) || (o.emit.scale && o.emit.ld % 4))
    throw std::runtime_error("conv_igemm: output strides must be multiples of 4");
  if (o.pool.psum) {
    const int pbn = conv_igemm_pool_cols(ks, IC, OC);
    const PoolPart& p = o.pool;
    const int ct = pbn - p.rpt;  // pooled channels per tile: a power of two from 4 to 64
    if (!pbn || OC % pbn || p.rpt < 0 || ct < 4 || ct > 64 || (ct & (ct - 1)) ||
        p.C != OC / pbn * (pbn - p.rpt) || !p.pmax ||
        !p.scale || !p.bias || !p.mask || o.colbias || o.rowmask || o.accumulate || o.yt || o.emit.scale || x_lo)
      throw std::runtime_error("conv_igemm: unsupported pooling partials");
  }
  const int M = B * HW, kind = igemm_kind(ks, IC, OC, split);
  if (prec == PREC_F16) igemm_dispatch<f16>(kind, x, x_lo, ldx, IC, w, icp, OC, o, M, s);
  else igemm_dispatch<bf16>(kind, x, x_lo, ldx, IC, w, icp, OC, o, M, s);
  KGX_CHECK_LAUNCH();
}

// Network input of one batch row and one group of 8 packed channels per workgroup (one thread per board point):
// the planes, float NCHW [nin][361], to compute-type NHWC rows of ldo channels (zero beyond nin, one 16-byte store
// per point), and, in the row's first group, the board statistics of launch_mask_prep: mask = plane 0, area = its
// sum, s1 = (sqrt(area) - 14) 0.1, s2 = (sqrt(area) - 14)^2 0.01 - 0.1. Workgroups (b, ldo / 8) compute the row's
// global-input bias of the stem instead (when `gl.W` is set). Groups of 8 channels spread the input's first touch
// over four times as many CUs as whole rows did (each CU's share of cache lines in flight is what its time waits on).
constexpr int IP_C = 32, IP_G = 32;  // the input packing's most planes (packed channels) and globals

template <typename T>
__global__ __launch_bounds__(384) void input_prep_kernel(const float* __restrict__ bin, int nin, T* __restrict__ out,
                                                         int ldo, float* __restrict__ mask, float* __restrict__ area,
                                                         float* __restrict__ s1, float* __restrict__ s2,
                                                         InputGlobal gl) {
  const int b = blockIdx.x, p = threadIdx.x, grp = blockIdx.y;
  // Every load is issued before any is used, from clamped (in-range) indices with no branch around it, so that a
  // thread waits for one round trip instead of one per load; the values past the real ones are then replaced.
  if (grp == ldo / 8) {
    // Up to IP_G globals in flight per output; the sum runs over i < nglob in order, as one multiply-add each.
    for (int o = p; o < gl.C; o += 384) {
      float g[IP_G], w[IP_G];
#pragma unroll
      for (int i = 0; i < IP_G; i++) {
        const int ic = min(i, gl.nglob - 1);
        g[i] = gl.glob[(size_t)b * gl.nglob + ic];
        w[i] = gl.W[(size_t)ic * gl.C + o];
      }
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < IP_G; i++)
        if (i < gl.nglob) acc += g[i] * w[i];
      gl.out[(size_t)b * gl.C + o] = acc;
    }
    return;
  }
  __shared__ float red[6];
  const int c0 = grp * 8;
  const float* src = bin + (size_t)b * nin * HW + min(p, HW - 1);
  float v[8];
#pragma unroll
  for (int c = 0; c < 8; c++) v[c] = src[(size_t)min(c0 + c, nin - 1) * HW];
#pragma unroll
  for (int c = 0; c < 8; c++)
    if (c0 + c >= nin) v[c] = 0.f;
  if (p < HW) {
    T t[8];
#pragma unroll
    for (int k = 0; k < 8; k++) t[k] = to_t<T>(v[k]);
    *(u32x4*)(out + ((size_t)b * HW + p) * ldo + c0) = *(const u32x4*)t;
  }
  if (grp != 0) return;
  float mk = 0.f;
  if (p < HW) {
    mk = v[0];
    mask[(size_t)b * HW + p] = mk;
  }
  float sum = mk;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if ((p & 63) == 0) red[p >> 6] = sum;
  __syncthreads();
  if (p == 0) {
    const float a = ((red[0] + red[1]) + (red[2] + red[3])) + (red[4] + red[5]);
    area[b] = a;
    const float c = sqrtf(a) - 14.f;
    s1[b] = c * 0.1f;
    s2[b] = c * c * 0.01f - 0.1f;
  }
}

void launch_input_prep(int prec, const float* bin, int nin, void* out, int ldo, float* mask, float* area, float* s1,
                       float* s2, int B, hipStream_t s, const InputGlobal& gl) {
  if (ldo % 8 != 0 || ldo < nin || ldo > IP_C || nin < 1)
    throw std::runtime_error("input_prep: bad packed channel count");
  if (gl.W && (!gl.glob || !gl.out || gl.C < 1 || gl.nglob < 1 || gl.nglob > IP_G))
    throw std::runtime_error("input_prep: bad global-input bias arguments");
  const dim3 grid(B, ldo / 8 + (gl.W ? 1 : 0));
  if (prec == PREC_F16)
    launch_k(input_prep_kernel<f16>, grid, 384, 0, s, bin, nin, (f16*)out, ldo, mask, area, s1, s2, gl);
  else if (prec == PREC_BF16)
    launch_k(input_prep_kernel<bf16>, grid, 384, 0, s, bin, nin, (bf16*)out, ldo, mask, area, s1, s2, gl);
  else throw std::runtime_error("input_prep: 16-bit only");
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
