// A nested-bottleneck junction in one launch: block k's exit 1x1 convolution (192 -> 384 channels, added into the
// trunk) and block k + 1's entry 1x1 convolution (384 -> 192), both on split 16-bit operands (hi*hi + lo*hi +
// hi*lo per product), over one 48-pixel tile per workgroup (bin2onnx.py:1263-1269: post(bnact(...)) into the trunk,
// then the next block's pre(bnact(x))).
//
// Between the two convolutions the separate kernels pass the trunk's next activation act(bn(x)) through memory as
// two 16-bit planes (4 bytes per value, written once and read once per junction). Here it stays in LDS: a workgroup
// computes all 384 trunk channels of its pixels, adds the trunk, stores the trunk once, and multiplies the
// activation it derives from it by the entry weights in place. Per pixel this moves 192 * 4 (the exit's operand) +
// 384 * 8 (the trunk read and written) + 192 * 6 (the inner stream and its 16-bit activation) bytes, against
// 3072 more for the two planes and their read-back. Both products take their weight fragments straight from
// memory into registers (packed in fragment order, one coalesced 1 KB load per fragment): every workgroup needs all
// 576 KB of them, which each XCD's L2 holds after the first touch.
//
// The arithmetic is that of the two separate implicit-GEMM kernels, in the same order: the exit's accumulator chain
// runs over its six 32-channel steps in order, each step lo*hi, hi*lo, hi*hi; the entry's twelve steps are summed
// in two chains, steps {0, 1, 4, 5, 8, 9} and {2, 3, 6, 7, 10, 11} (the separate kernel's two wave groups over its
// 128-channel stages), then added; the epilogues are the same expressions. So the junction's outputs equal the
// separate kernels' bit for bit.
//
// The stem junction (STEM) is the same launch with the network's stem in place of the exit: a 3x3 convolution of
// the packed input planes (at most 32 channels, 16-bit operands, one plane) into the trunk, with the row's global
// bias added (bin2onnx.py:1466-1492), then the first nested block's entry 1x1. Its nine taps are nine steps in tap
// order over the 48-pixel tile's rows and their 20-row halo, staged in LDS, as the separate kernel sums them.
#include "kgx_device.h"

#include <vector>

namespace kgx {

namespace {

constexpr int JCI = kJunctionInner, JCO = kJunctionOuter;
constexpr int JR = 48;                         // pixels per workgroup (three 16-row MFMA blocks)
constexpr int JNT = 512;                       // threads: eight waves, two per SIMD
constexpr int K1 = JCI / 32, K2 = JCO / 32;    // 16x16x32 steps of the exit and the entry product
constexpr int CB1 = JCO / 16;                  // 16-column blocks of the exit's output
constexpr int FRAG = 64 * 8;                   // elements per packed fragment (64 lanes x 8)
constexpr int W2OFF = CB1 * K1 * 2 * FRAG;     // the entry's fragments follow the exit's
// The entry's outputs NO: a nested block's 192 (kJunctionInner), or the heads' p1 | g1 | v1 convolution's 96
// (kJunctionHead) after the trunk's last exit.
__host__ __device__ constexpr int junction_welems(int no) { return W2OFF + (no / 16) * K2 * 2 * FRAG; }
// LDS: the entry's operand (the activation planes, [64-channel slice][plane][pixel][128 bytes], 16-byte chunks
// swizzled as chunk ^ (pixel / 2 % 8)), then one region that holds in turn the exit's operand (same layout over
// 192 channels), the exit's float tile [48][384 + 4] and the entry's two float tiles [2][48][NO + 4] (at most
// the exit's).
constexpr int LD1 = JCO + 4;
constexpr int ACTB = (JCO / 64) * 2 * JR * 128;
constexpr int A1B = (JCI / 64) * 2 * JR * 128, C1B = JR * LD1 * 4, C2B = 2 * JR * (JCI + 4) * 4;
constexpr int R1B = A1B > C1B ? (A1B > C2B ? A1B : C2B) : (C1B > C2B ? C1B : C2B);
constexpr int LDSB = ACTB + R1B;
// Epilogue mappings, the same for every thread (no branch around a memory access, so the compiler's count of the
// loads in flight stays exact and a later wait for a prefetched weight fragment leaves the trunk's stores in
// flight): thread t takes channel quads t % G + G q, q < 3, of pixels t / G + R e, for the exit's G = 32 and R = 16
// (three pixels each) and the entry's G = NO / 12 and R = 512 / G (pixels past 48 skipped at the end). Consecutive
// lanes take consecutive quads, so each access of a wave covers whole cache lines.
constexpr int E1 = 3;
constexpr int NS = 2;  // weight steps in flight per product (of six per wave)
static_assert(JNT / 64 == 8 && CB1 == 3 * 8 && K2 == 12, "wave layout assumes 384 and 192 channels");

// The XCD-aware tile order: workgroup g runs on XCD g % 8, and the four 48-pixel tiles of one 192-pixel region go
// to that region's XCD (region r on XCD r % 8), as every 192-pixel convolution around the junction maps it, so the
// junction reads its operand from the L2 its producer wrote and its consumer reads the junction's output there.
__host__ __device__ inline int junction_tile(int g) {
  const int xcd = g & 7, slot = g >> 3;
  return 4 * (xcd + 8 * (slot >> 2)) + (slot & 3);
}

// Waits for this wave's LDS accesses, then for every wave: nothing else. A fence (__syncthreads()) would also wait
// for the wave's loads and stores in flight (the weight prefetch, the trunk's stores). The compiler moves no memory
// access across the clobbers, nor the clobbers across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// The stem's packed fragments: [column block][tap] single-plane fragments, then the entry's.
constexpr int KS3 = 9;                       // the stem's steps: one per tap, 32 channels each
constexpr int W2STEM = CB1 * KS3 * FRAG;
constexpr int SR = JR + 40, SRB = 80;        // the stem's staged pixel rows (tile and halos), bytes per LDS row

// ACT1: the exit's emission activation (ACT_MISH), or -1: the one eo names, chosen per value at run time. NO: the
// entry's outputs (192 or 96). A trunk that ends here (eo.y_dead) is read and not stored. STEM: the exit is the
// network's stem (X: packed input rows of ldx <= 32 channels; eo adds the row's global bias, eo.colbias, instead of
// a residual). SC2 >= 0: the entry's store case (store_flags of no: SF_Y | SF_EMIT emitting mish, or SF_Y), fixed by
// the launch so that the kernel holds only that store path; -1: chosen from the arguments.
template <typename T, int ACT1, int NO, bool STEM, int SC2 = -1>
__global__ __launch_bounds__(JNT, 1) void junction_kernel(const T* __restrict__ X, const T* __restrict__ Xlo, int ldx,
                                                          const T* __restrict__ W, int M, ConvOut eo, ConvOut no) {
  typedef typename std::conditional<std::is_same<T, f16>::value, half8, bf16x8>::type frag_t;
  static_assert(NO == 192 || NO == 96, "entry outputs");
  constexpr int W2 = STEM ? W2STEM : W2OFF;  // the entry's fragments
  constexpr int CB2 = NO / 16, LD2 = NO + 4;
  constexpr int G2 = NO / 12, R2 = JNT / G2, E2 = (JR + R2 - 1) / R2;  // the entry epilogue's mapping
  __shared__ __align__(1024) char smem[LDSB];
  char* const act = smem;
  char* const r1 = smem + ACTB;
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int m0 = junction_tile(blockIdx.x) * JR;
  if (m0 >= M) {  // an idle workgroup still touches its share of the next launch's weights
    l2_touch_keep(l2_touch(no.pf, no.pf_bytes, tid));
    return;
  }

  auto mfma = [](const frag_t& a, const frag_t& b, floatx4 c) {
    if constexpr (std::is_same<T, f16>::value) return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  };
  // Packed weight fragment (column block cb, step ks of K, plane pl): lane l holds w[16 cb + l % 16][32 ks + 8 (l / 16)
  // .. + 8], the MFMA's B operand.
  auto wfrag = [&](int base, int cb, int K, int ks, int pl) {
    return *(const frag_t*)(W + base + ((cb * K + ks) * 2 + pl) * FRAG + lane * 8);
  };
  // A operand of 16-pixel block i at step ks, plane pl, from an LDS operand: lane l holds pixel 16 i + l % 16,
  // channels 32 ks + 8 (l / 16) .. + 8 (the block's pixels share one swizzle, that of l % 16).
  auto afrag = [&](const char* base, int i, int ks, int pl) {
    const int chunk = ((ks & 1) * 4 + g4) ^ ((r16 >> 1) & 7);
    return *(const frag_t*)(base + (((ks >> 1) * 2 + pl) * JR + 16 * i + r16) * 128 + chunk * 16);
  };

  // The exit epilogue's inputs: the trunk values it adds to (the stem: the row's global bias), the emission's scale,
  // bias and board mask (channels c1 + 128 q .. + 3 of pixels p1 + 16 e; rows past M read row M - 1, never
  // stored). They are issued after the product's last weight loads (a wait covers every load issued before the one
  // it waits for), in flight during its last steps.
  const int c1 = 4 * (tid & 31), p1 = tid >> 5;
  floatx4 yres[E1][3], es1[3], eb1[3];
  float mk1[E1];
  auto load_epi1 = [&]() {
#pragma unroll
    for (int e = 0; e < E1; e++) {
      const int m = min(m0 + p1 + 16 * e, M - 1);
#pragma unroll
      for (int q = 0; q < 3; q++)
        yres[e][q] = STEM ? *(const floatx4*)(eo.colbias + (size_t)(m / HW) * eo.ld_colbias + c1 + 128 * q)
                          : *(const floatx4*)(eo.y + (size_t)m * eo.ldy + c1 + 128 * q);
      mk1[e] = eo.emit.mask[m];
    }
#pragma unroll
    for (int q = 0; q < 3; q++) {
      es1[q] = *(const floatx4*)(eo.emit.scale + c1 + 128 * q);
      eb1[q] = *(const floatx4*)(eo.emit.bias + c1 + 128 * q);
    }
  };

  floatx4 acc[3][3];
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (STEM) {
    // The stem, wave wv: output columns 48 wv .. + 48 (blocks 3 wv + j), all 48 pixels, over the nine taps in order
    // (one 16x16x32 step each: 32 channels, those past ldx zero). The pixel rows [m0 - 20, m0 + 68) go into LDS
    // (rows off the batch and channels past ldx as zeros, from loads of clamped rows) while the ring's first
    // weights are in flight.
    const int sr = tid >> 2, sc = tid & 3, sg = m0 - 20 + sr;
    const u32x4 rv = *(const u32x4*)(X + (size_t)min(max(sg, 0), M - 1) * ldx + (8 * sc < ldx ? 8 * sc : 0));
    frag_t b1[NS][3];
    auto load_b1 = [&](int slot, int t) {
#pragma unroll
      for (int j = 0; j < 3; j++) b1[slot][j] = *(const frag_t*)(W + ((3 * wv + j) * KS3 + t) * FRAG + lane * 8);
    };
#pragma unroll
    for (int k = 0; k < NS; k++) load_b1(k, k);
    const bool sok = sg >= 0 && sg < M && 8 * sc < ldx;
    if (tid < SR * 4) *(u32x4*)(r1 + sr * SRB + sc * 16) = sok ? rv : u32x4{0, 0, 0, 0};
    else if (tid < SR * 4 + SRB / 16) *(u32x4*)(r1 + SR * SRB + (tid - SR * 4) * 16) = u32x4{0, 0, 0, 0};  // zero row
    // Tap validity of this lane's pixels (bit t: the neighbour at tap t is on the board); off-board neighbours,
    // and pixels past M, read the zero row.
    unsigned vmask[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int m = m0 + 16 * i + r16;
      unsigned bits = 0;
      if (m < M) {
        const int pt = m % HW, y = pt / POS, x = pt - y * POS;
#pragma unroll
        for (int t = 0; t < KS3; t++)
          if ((unsigned)(y + t / 3 - 1) < (unsigned)POS && (unsigned)(x + t % 3 - 1) < (unsigned)POS) bits |= 1u << t;
      }
      vmask[i] = bits;
    }
    lds_barrier();
    frag_t a[2][3];
    auto load_a = [&](int set, int t) {
      const int shift = (t / 3 - 1) * POS + (t % 3 - 1);
#pragma unroll
      for (int i = 0; i < 3; i++) {
        const int row = (vmask[i] >> t) & 1 ? 16 * i + r16 + 20 + shift : SR;
        a[set][i] = *(const frag_t*)(r1 + row * SRB + g4 * 16);
      }
    };
    load_a(0, 0);
#pragma unroll
    for (int t = 0; t < KS3; t++) {
      if (t + 1 < KS3) load_a((t + 1) & 1, t + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) acc[i][j] = mfma(a[t & 1][i], b1[t % NS][j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + NS < KS3) load_b1(t % NS, t + NS);
      if (t + NS + 1 == KS3) load_epi1();
    }
  } else {
    // Exit product, wave wv: output columns 48 wv .. + 48 (blocks 3 wv + j), all 48 pixels. Its weight fragments go
    // through a ring of NS steps, the first NS loaded while the operand's direct loads are in flight (the wait for
    // those covers them too), so that the weights stream from L2 in the time that would otherwise only wait.
    frag_t b1[NS][3][2];
    auto load_b1 = [&](int slot, int ks) {
#pragma unroll
      for (int j = 0; j < 3; j++)
#pragma unroll
        for (int pl = 0; pl < 2; pl++) b1[slot][j][pl] = wfrag(0, 3 * wv + j, K1, ks, pl);
    };
#pragma unroll
    for (int k = 0; k < NS; k++) load_b1(k, k);
    // The exit's operand straight into LDS: 36 loads of 8 pixel rows x 128 bytes (64-channel slice kp, plane pl,
    // rows 8 grp ..), lane i filling row 8 grp + i / 8 at stored chunk i % 8 from source chunk (i % 8) ^ swizzle.
    // Rows past M lie beyond the buffer range and read as zero.
    {
      const int rb = ldx * (int)sizeof(T), nbytes = min(JR, M - m0) * rb;
      const T* xb = X + (size_t)m0 * ldx;
      const T* xlb = Xlo + (size_t)m0 * ldx;
#pragma unroll
      for (int u = 0; u < 5; u++) {
        const int q = u * 8 + wv;
        if (q < 36) {
          const int kp = q / 12, pl = (q / 6) & 1, grp = q % 6;
          const int row = grp * 8 + (lane >> 3), sc = (lane & 7) ^ ((row >> 1) & 7);
          lds_load16(pl ? xlb : xb, nbytes, r1 + ((kp * 2 + pl) * JR + grp * 8) * 128, row * rb + kp * 128 + sc * 16);
        }
      }
    }
    // The direct loads are not counted by the compiler: wait for all of this wave's loads, then for every wave.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    {
      frag_t ah[2][3], al[2][3];
      auto load_a1 = [&](int set, int ks) {
#pragma unroll
        for (int i = 0; i < 3; i++) {
          ah[set][i] = afrag(r1, i, ks, 0);
          al[set][i] = afrag(r1, i, ks, 1);
        }
      };
      load_a1(0, 0);
#pragma unroll
      for (int ks = 0; ks < K1; ks++) {
        const int s = ks & 1;
        if (ks + 1 < K1) load_a1(s ^ 1, ks + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) acc[i][j] = mfma(al[s][i], b1[ks % NS][j][0], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) acc[i][j] = mfma(ah[s][i], b1[ks % NS][j][1], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) acc[i][j] = mfma(ah[s][i], b1[ks % NS][j][0], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
        if (ks + NS < K1) load_b1(ks % NS, ks + NS);
        if (ks + NS + 1 == K1) load_epi1();
      }
    }
  }

  // Entry product, wave wv: step chain kg = wv / 4 (steps 2 kg + 4 (p / 2) + p % 2), output columns 48 cg .. + 48
  // (blocks 3 cg + j, cg = wv % 4), all 48 pixels. Its first NS steps' weights load after the exit's float tile is
  // in LDS and ahead of the trunk's stores (the wait for a load also waits for the stores issued before it), in
  // flight during the exit epilogue.
  // (With 96 outputs, waves with cg >= 2 repeat the columns of cg - 2 and do not write them: every wave then issues
  // the same instructions.)
  const int kg = wv >> 2, cg = (wv & 3) % (CB2 / 3);
  const bool c2own = (wv & 3) < CB2 / 3;
  auto kstep = [&](int p) { return 2 * kg + 4 * (p >> 1) + (p & 1); };
  frag_t b2[NS][3][2];
  auto load_b2 = [&](int slot, int p) {
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int pl = 0; pl < 2; pl++) b2[slot][j][pl] = wfrag(W2, 3 * cg + j, K2, kstep(p), pl);
  };
  // The exit's float tile over its operand's LDS (every wave is done reading the operand first).
  lds_barrier();
  float* const C1 = (float*)r1;
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) C1[(16 * i + 4 * g4 + r) * LD1 + 48 * wv + 16 * j + r16] = acc[i][j][r];
#pragma unroll
  for (int k = 0; k < NS; k++) load_b2(k, k);
  // The entry epilogue's per-channel inputs (channels c2 + 4 G2 q .. + 3 of pixels p2 + R2 e), loaded during the
  // entry product's last block.
  const int c2 = 4 * (tid % G2), p2 = tid / G2;
  const int fl2 = store_flags(no);
  floatx4 es2[3], eb2[3];
  float mk2[E2];
  const float* const es2p = no.emit.scale ? no.emit.scale : eo.emit.scale;  // (any readable floats when unused)
  const float* const eb2p = no.emit.scale ? no.emit.bias : eo.emit.bias;
  const float* const mk2p = no.emit.scale ? no.emit.mask : eo.emit.mask;
  auto load_epi2 = [&]() {
#pragma unroll
    for (int q = 0; q < 3; q++) {
      es2[q] = *(const floatx4*)(es2p + c2 + 4 * G2 * q);
      eb2[q] = *(const floatx4*)(eb2p + c2 + 4 * G2 * q);
    }
#pragma unroll
    for (int e = 0; e < E2; e++) mk2[e] = mk2p[min(m0 + p2 + R2 * e, M - 1)];
  };

  lds_barrier();

  // Exit epilogue: the trunk plus the product, stored; the activation act(x * scale + bias) * mask in its two
  // 16-bit planes (the high part, and the rounding of what it leaves) into the entry's LDS operand. The trunk goes
  // out through a buffer whose range ends at row M, so rows past it are dropped without a branch. It runs in three
  // channel groups q (channels c1 + 128 q: the operand's 64-channel slices 2 q and 2 q + 1), and the entry product
  // in three blocks of two steps, block b reading slices 2 b (chain 0) and 2 b + 1 (chain 1): group q + 1's VALU
  // work follows block q's MFMAs in each wave's instruction stream, so that it issues while they run, and a
  // barrier separates the groups. The accumulation order stays that of the separate kernel.
  // (A trunk that ends here gets an empty range: its stores are all dropped.)
  const auto ybuf = __builtin_amdgcn_make_buffer_rsrc(
      eo.y + (size_t)m0 * eo.ldy, 0, eo.y_dead ? 0 : min(JR, M - m0) * eo.ldy * (int)sizeof(float), 0x00020000);
  // Pixel row e of group q; A >= 0 the emission's activation known here, -1 chosen at run time.
  auto epi1 = [&](auto act_c, int q, int e) {
    constexpr int A = decltype(act_c)::value;
    const int p = p1 + 16 * e, n = c1 + 128 * q;
    floatx4 v = *(const floatx4*)(C1 + p * LD1 + n);
    v += yres[e][q];
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ybuf, (p * eo.ldy + n) * 4, 0, 2);
    float t[4], l[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float a = v[k] * es1[q][k] + eb1[q][k];
      if constexpr (A >= 0) t[k] = act_f<A>(a) * mk1[e];
      else t[k] = act_rt(a, eo.emit.act) * mk1[e];
      l[k] = t[k] - (float)to_t<T>(t[k]);
    }
    T hi[4] = {to_t<T>(t[0]), to_t<T>(t[1]), to_t<T>(t[2]), to_t<T>(t[3])};
    T lo[4] = {to_t<T>(l[0]), to_t<T>(l[1]), to_t<T>(l[2]), to_t<T>(l[3])};
    const int kp = n >> 6, chunk = ((n & 63) >> 3) ^ ((p >> 1) & 7);
    char* d = act + ((kp * 2) * JR + p) * 128 + chunk * 16 + (n & 7) * (int)sizeof(T);
    *(uint2*)d = *(const uint2*)hi;
    *(uint2*)(d + JR * 128) = *(const uint2*)lo;
  };

  floatx4 acc2[3][3];
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) acc2[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  frag_t ah[2][3], al[2][3];
  auto load_a2 = [&](int set, int p) {
#pragma unroll
    for (int i = 0; i < 3; i++) {
      ah[set][i] = afrag(act, i, kstep(p), 0);
      al[set][i] = afrag(act, i, kstep(p), 1);
    }
  };
  auto mma2 = [&](int p) {
    const int s = p & 1;
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
      for (int j = 0; j < 3; j++) acc2[i][j] = mfma(al[s][i], b2[p % NS][j][0], acc2[i][j]);
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
      for (int j = 0; j < 3; j++) acc2[i][j] = mfma(ah[s][i], b2[p % NS][j][1], acc2[i][j]);
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
      for (int j = 0; j < 3; j++) acc2[i][j] = mfma(ah[s][i], b2[p % NS][j][0], acc2[i][j]);
  };
  int pfv;
  // The entry epilogue's path: a specialized store (which loads nothing more), or the general one.
  const bool fast = SC2 >= 0 || (fl2 == (SF_Y | SF_EMIT) && no.emit.act == ACT_MISH);
  auto run = [&](auto act_c) {
#pragma unroll
    for (int e = 0; e < E1; e++) epi1(act_c, 0, e);
    lds_barrier();
#pragma unroll
    for (int b = 0; b < 3; b++) {
      if (b == 2) {
        load_epi2();
        // The next launch's weights into this XCD's L2 during the last steps (after every load this kernel waits
        // for, so that no wait includes it; the general epilogue path loads more, and a wait for those would).
        pfv = l2_touch(no.pf, fast ? no.pf_bytes : 0, tid);
      }
      load_a2(0, 2 * b);
      __builtin_amdgcn_sched_barrier(0);
      mma2(2 * b);
      load_a2(1, 2 * b + 1);
      if (b < 2) {
        epi1(act_c, b + 1, 0);
        epi1(act_c, b + 1, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (2 * b + NS < K2 / 2) load_b2(0, 2 * b + NS);
      mma2(2 * b + 1);
      if (b < 2) epi1(act_c, b + 1, 2);
      __builtin_amdgcn_sched_barrier(0);
      if (2 * b + 1 + NS < K2 / 2) load_b2(1, 2 * b + 1 + NS);
      if (b < 2) lds_barrier();
    }
  };
  run(std::integral_constant<int, ACT1>{});

  // The two chains' float tiles over the exit's (whose last reads preceded the barrier above).
  float* const C2 = (float*)r1;
  if (c2own) {
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
      for (int j = 0; j < 3; j++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          C2[(kg * JR + 16 * i + 4 * g4 + r) * LD2 + 48 * cg + 16 * j + r16] = acc2[i][j][r];
  }
  lds_barrier();

  // Entry epilogue: chain 0 plus chain 1, then the convolution's outputs (the inner stream and its consumer's
  // activation) as the separate kernel stores them. At the end of the kernel, so these stores may branch.
#pragma unroll
  for (int e = 0; e < E2; e++) {
    const int p = p2 + R2 * e, m = m0 + p;
    if (p < JR && m < M) {
#pragma unroll
      for (int q = 0; q < 3; q++) {
        const int n = c2 + 4 * G2 * q;
        floatx4 sum = *(const floatx4*)(C2 + p * LD2 + n);
        sum += *(const floatx4*)(C2 + (JR + p) * LD2 + n);
        if constexpr (SC2 == SF_Y) {
          conv_store4<T, ACT_ID, SF_Y>(no, m, n, sum, floatx4{0.f, 0.f, 0.f, 0.f}, 1.f, es2[q], eb2[q], mk2[e]);
        } else if (SC2 == (SF_Y | SF_EMIT) || fast) {
          conv_store4<T, ACT_MISH, SF_Y | SF_EMIT>(no, m, n, sum, floatx4{0.f, 0.f, 0.f, 0.f}, 1.f, es2[q], eb2[q],
                                                   mk2[e]);
        } else if constexpr (SC2 < 0) {
          const floatx4 yacc = (fl2 & SF_ACC) ? *(const floatx4*)(no.y + (size_t)m * no.ldy + n)
                                              : floatx4{0.f, 0.f, 0.f, 0.f};
          conv_store4<T>(no, m, n, sum, yacc, (fl2 & SF_ROWMASK) ? no.rowmask[m] : 1.f, es2[q], eb2[q], mk2[e]);
        }
      }
    }
  }
  l2_touch_keep(pfv);
}

}  // namespace

int junction_tile_of(int g) { return junction_tile(g); }

int junction_grid(int M) {
  const int regions = (M + 4 * JR - 1) / (4 * JR);
  return 32 * ((regions + 7) / 8);
}

// Fragment (cb, ks, plane) of a K-step weight matrix w [cols][32 K] at `base`: lane l, element e holds column
// 16 cb + l % 16, channel 32 ks + 8 (l / 16) + e; the low plane holds w - round(w).
static void pack_split(const float* w, int cbs, int K, size_t base, int prec, std::vector<float>& out) {
  for (int cb = 0; cb < cbs; cb++)
    for (int ks = 0; ks < K; ks++)
      for (int l = 0; l < 64; l++)
        for (int e = 0; e < 8; e++) {
          const float v = w[(size_t)(16 * cb + l % 16) * (32 * K) + 32 * ks + 8 * (l / 16) + e];
          const size_t at = base + (size_t)((cb * K + ks) * 2) * FRAG + l * 8 + e;
          out[at] = v;
          out[at + FRAG] = v - conv_round_operand(v, prec);
        }
}

void junction_pack_weights(const float* w_exit, const float* w_entry, int entry_oc, int prec, std::vector<float>& out) {
  if (entry_oc != kJunctionInner && entry_oc != kJunctionHead) throw std::runtime_error("junction: entry outputs");
  out.assign(junction_welems(entry_oc), 0.f);
  pack_split(w_exit, CB1, K1, 0, prec, out);
  pack_split(w_entry, entry_oc / 16, K2, W2OFF, prec, out);
}

int stem_junction_welems(int no) { return W2STEM + (no / 16) * K2 * 2 * FRAG; }

void stem_junction_pack_weights(const float* w_stem, int ic, const float* w_entry, int entry_oc, int prec,
                                std::vector<float>& out) {
  if (entry_oc != kJunctionInner) throw std::runtime_error("stem junction: entry outputs");
  if (ic < 1 || ic > 32) throw std::runtime_error("stem junction: at most 32 input channels");
  out.assign(stem_junction_welems(entry_oc), 0.f);
  // Stem fragment (cb, t), one plane: lane l, element e holds w[16 cb + l % 16][8 (l / 16) + e][t] (zero past ic).
  for (int cb = 0; cb < CB1; cb++)
    for (int t = 0; t < KS3; t++)
      for (int l = 0; l < 64; l++)
        for (int e = 0; e < 8; e++) {
          const int ch = 8 * (l / 16) + e;
          out[(size_t)(cb * KS3 + t) * FRAG + l * 8 + e] =
              ch < ic ? w_stem[((size_t)(16 * cb + l % 16) * ic + ch) * KS3 + t] : 0.f;
        }
  pack_split(w_entry, entry_oc / 16, K2, W2STEM, prec, out);
}

void launch_junction(int prec, const void* x, const void* x_lo, int ldx, const void* w, const ConvOut& eo,
                     const ConvOut& no, int entry_oc, int B, hipStream_t s) {
  if (prec != PREC_F16 && prec != PREC_BF16) throw std::runtime_error("junction: 16-bit operands only");
  if (entry_oc != kJunctionInner && entry_oc != kJunctionHead) throw std::runtime_error("junction: entry outputs");
  if (B <= 0) return;
  if (!x || !x_lo || !w || ldx < JCI || ldx % 8 || ((uintptr_t)x | (uintptr_t)x_lo | (uintptr_t)w) % 16)
    throw std::runtime_error("junction: operands must be 16-byte aligned rows of at least 192 channels");
  // The exit's output is the trunk's residual add (stored, or read only where the trunk ends) and the emission of
  // the entry's activation, nothing else.
  if (!eo.y || !eo.accumulate || eo.ldy % 4 || eo.yt || eo.rowmask || eo.colbias || !eo.emit.scale ||
      !eo.emit.bias || !eo.emit.mask || eo.pool.psum || ((uintptr_t)eo.y | (uintptr_t)eo.emit.scale |
                                                         (uintptr_t)eo.emit.bias) % 16)
    throw std::runtime_error("junction: the exit must add into the trunk and emit the entry's activation");
  if (no.pool.psum || (no.y && (no.ldy % 4 || (uintptr_t)no.y % 16)) || (no.yt && no.ldyt % 4) ||
      (no.colbias && no.ld_colbias % 4) || (no.emit.scale && (no.emit.ld % 4 || (uintptr_t)no.emit.scale % 16 ||
                                                              (uintptr_t)no.emit.bias % 16)))
    throw std::runtime_error("junction: unsupported entry outputs");
  const int M = B * HW;
  const bool mish = eo.emit.act == ACT_MISH;
  // The entry's store case for a kernel that holds only that store path (the networks' two), else -1.
  const int fl2 = store_flags(no);
  const int sc2 = !mish ? -1
                  : entry_oc == kJunctionInner && fl2 == (SF_Y | SF_EMIT) && no.emit.act == ACT_MISH ? SF_Y | SF_EMIT
                  : entry_oc == kJunctionHead && fl2 == SF_Y ? SF_Y : -1;
  auto go = [&](auto tc, auto noc) {
    typedef decltype(tc) TT;
    constexpr int N = decltype(noc)::value;
    constexpr int SPEC2 = N == kJunctionInner ? SF_Y | SF_EMIT : SF_Y;
    launch_k(!mish ? junction_kernel<TT, -1, N, false>
                   : sc2 >= 0 ? junction_kernel<TT, ACT_MISH, N, false, SPEC2> : junction_kernel<TT, ACT_MISH, N, false>,
             junction_grid(M), JNT, 0, s, (const TT*)x, (const TT*)x_lo, ldx, (const TT*)w, M, eo, no);
  };
  typedef std::integral_constant<int, kJunctionInner> Inner;
  typedef std::integral_constant<int, kJunctionHead> Head;
  if (prec == PREC_F16) {
    if (entry_oc == kJunctionInner) go(f16(), Inner());
    else go(f16(), Head());
  } else {
    if (entry_oc == kJunctionInner) go(bf16(), Inner());
    else go(bf16(), Head());
  }
  KGX_CHECK_LAUNCH();
}

void launch_stem_junction(int prec, const void* x, int ldx, const void* w, const ConvOut& eo, const ConvOut& no,
                          int B, hipStream_t s) {
  if (prec != PREC_F16 && prec != PREC_BF16) throw std::runtime_error("stem junction: 16-bit operands only");
  if (B <= 0) return;
  if (!x || !w || ldx < 8 || ldx > 32 || ldx % 8 || ((uintptr_t)x | (uintptr_t)w) % 16)
    throw std::runtime_error("stem junction: packed input rows of 8 to 32 channels, 16-byte aligned");
  // The stem's output is the trunk (stored), its row bias and the emission of the entry's activation, nothing else.
  if (!eo.y || eo.accumulate || eo.y_dead || eo.ldy % 4 || eo.yt || eo.rowmask || !eo.colbias || eo.ld_colbias % 4 ||
      !eo.emit.scale || !eo.emit.bias || !eo.emit.mask || eo.pool.psum ||
      ((uintptr_t)eo.y | (uintptr_t)eo.colbias | (uintptr_t)eo.emit.scale | (uintptr_t)eo.emit.bias) % 16)
    throw std::runtime_error("stem junction: the stem must store the trunk with its row bias and emit the entry's "
                             "activation");
  if (no.pool.psum || (no.y && (no.ldy % 4 || (uintptr_t)no.y % 16)) || (no.yt && no.ldyt % 4) ||
      (no.colbias && no.ld_colbias % 4) || (no.emit.scale && (no.emit.ld % 4 || (uintptr_t)no.emit.scale % 16 ||
                                                              (uintptr_t)no.emit.bias % 16)))
    throw std::runtime_error("stem junction: unsupported entry outputs");
  const int M = B * HW;
  const bool mish = eo.emit.act == ACT_MISH;
  const bool spec2 = mish && store_flags(no) == (SF_Y | SF_EMIT) && no.emit.act == ACT_MISH;
  auto go = [&](auto tc) {
    typedef decltype(tc) TT;
    launch_k(!mish ? junction_kernel<TT, -1, kJunctionInner, true>
                   : spec2 ? junction_kernel<TT, ACT_MISH, kJunctionInner, true, SF_Y | SF_EMIT>
                           : junction_kernel<TT, ACT_MISH, kJunctionInner, true>,
             junction_grid(M), JNT, 0, s, (const TT*)x, (const TT*)x, ldx, (const TT*)w, M, eo, no);
  };
  if (prec == PREC_F16) go(f16());
  else go(bf16());
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
