// Host-side declarations of the kernel launchers (kgx_kernels.hip). Every launcher enqueues one kernel on
// `stream` and returns without waiting.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <vector>

#include "kgx.h"

namespace kgx {

constexpr int POS = 19;
constexpr int HW = POS * POS;             // board points per row

enum Prec { PREC_F32 = 0, PREC_F16 = 1, PREC_BF16 = 2 };
enum Act { ACT_ID = 0, ACT_RELU = 1, ACT_MISH = 2, ACT_SILU = 3 };

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Batch-norm + activation + board-mask prologue applied to a convolution's input as it is loaded:
// a = (x + prebias[b][c]) * scale[c] + bias[c]; x' = act(a) * mask[b][pos]. scale == nullptr disables it.
struct Prologue {
  const float* scale = nullptr;
  const float* bias = nullptr;
  const float* prebias = nullptr;  // [B][ld_prebias] or null
  int ld_prebias = 0;
  int act = ACT_ID;
  const float* mask = nullptr;     // [B*HW]
};

// Activation of a consumer layer, written by the producer's epilogue from its final float output y[m][n]:
// out[m][n] = T(act(y * scale[n] + bias[n]) * mask[m]). scale == nullptr disables it. With out_lo set the
// activation a is written as two compute-type operands, out = T(a) and out_lo = T(a - T(a)) (same layout), for a
// consumer that multiplies with split operands (a float-accurate convolution on 16-bit matrix cores).
struct Emit {
  const float* scale = nullptr;
  const float* bias = nullptr;
  int act = ACT_ID;
  const float* mask = nullptr;
  void* out = nullptr;
  void* out_lo = nullptr;
  int ld = 0;
};

// Board pooling partials of an implicit-GEMM convolution's pooled branch (a global-pooling block's gpool
// channels), computed in the epilogue. The convolution's weights interleave the branches per column tile of BN
// outputs (conv_igemm_pool_cols): tile t's first `rpt` columns are regular channels t * rpt + j, stored to y as
// usual (y holds the regular channels only, in their own order); its other BN - rpt columns are pooled channels
// c = t * (BN - rpt) + j, which are not stored. Every workgroup thus carries an equal share of the pooling. Per
// tile of BM pixels mt (conv_igemm_tile_rows) and segment s (0: the batch row of the tile's first pixel, 1: the
// next row, when the tile reaches into it),
//   psum[(mt * 2 + s) * C + c] = sum of round(x * 2^24) over the segment's pixels (64-bit integers: exact, so a
//                                row's sum does not depend on how its tiles cut it, i.e. on its batch position),
//   pmax[(mt * 2 + s) * C + c] = max of x + (mask[m] * 1e4 - 1e4),
// with x = act(v * scale[c] + bias[c]) * mask[m]. Requires rpt a multiple of 4, (BN - rpt) / 4 a power of two up
// to 16, C = (OC / BN) (BN - rpt), and no colbias, rowmask, residual, compute-type copy or emission.
constexpr float kPoolFix = 16777216.f;  // 2^24: the fixed-point scale of the partial sums
struct PoolPart {
  long long* psum = nullptr;
  float* pmax = nullptr;
  const float* scale = nullptr; const float* bias = nullptr; int act = ACT_ID;
  const float* mask = nullptr;
  int rpt = 0, C = 0;
};

// The 128-byte line of the next op's weights (ConvOut::pf) that thread tid of workgroup g of a grid-workgroup launch
// touches (l2_touch): workgroup g runs on XCD g mod 8, and the n workgroups of that XCD take lines s + n tid, s =
// g / 8, so the XCD touches each of its first n x threads lines once.
__host__ __device__ inline int l2_touch_line(int g, int grid, int tid) {
  return (g >> 3) + ((grid - (g & 7) + 7) >> 3) * tid;
}

// Output of a convolution or GEMM, element (m, n) with accumulated value v:
// v += colbias[m / HW][n]; v *= rowmask[m]; yt = T(v); y = (accumulate ? y : 0) + v; then the emission from y.
struct ConvOut {
  float* y = nullptr; int ldy = 0;
  bool accumulate = false;
  bool y_dead = false;  // y (and the residual, when accumulating) is read but the result is not stored: the
                        // stream ends here and only the emission consumes it
  const float* colbias = nullptr; int ld_colbias = 0;
  const float* rowmask = nullptr;
  void* yt = nullptr; int ldyt = 0;
  Emit emit;
  PoolPart pool;  // implicit-GEMM convolutions only
  // The weights of the launch that follows (pf_bytes bytes; null: none), which the implicit-GEMM and junction
  // kernels touch into their XCDs' L2 during their epilogue, one 4-byte load per 128-byte line, so that the next
  // launch reads them from L2 instead of MALL.
  const char* pf = nullptr; int pf_bytes = 0;
};

// Winograd F(tm x tm, 3x3), tm = 4 (36 tile points, 25 tiles per board) or 2 (16 points, 100 tiles).
// Transformed inputs are tile-major: V[t][point][c_pad].
int wino_tiles(int tm);
int wino_points(int tm);

// Winograd input transform of an activation x: compute-type NHWC rows of `ldx` (the consumer activation written
// by the producer), or float NCHW when `nchw_f32` (the network input).
void launch_wino_in(int prec, int tm, const void* x, int ldx, bool nchw_f32, void* V, int B, int C, int c_pad,
                    hipStream_t s);

// F(4x4,3x3) output transform of the point GEMMs M[t][point][oc_pad] (float) into `o`.
void launch_wino_out(int prec, int tm, const float* M, int oc_pad, int OC, const ConvOut& o, int B, hipStream_t s);

// F(2x2,3x3) point GEMMs fused with the output transform: V [t_pad][16][icp], U [16][ocp][icp] -> `o`.
void launch_wino2_fused(int prec, const void* V, const void* U, int t_pad, int icp, int ocp, int OC, const ConvOut& o,
                        int B, hipStream_t s);

// Filter transform G g G^T of w [oc][ic][3][3] into U[points][oc_pad][ic_pad] (host, double precision).
void wino_filter_host(int tm, const float* w, int oc, int ic, int oc_pad, int ic_pad, float* U);

// C[z] = A[z] * Bt[z]^T on MFMA: A [M][K] (row stride lda; T, or float with a prologue), Bt [N][K].
// Batch z offsets: A sA, Bt sB, outputs sC (elements, applied to out.y / out.yt).
// Epilogue of the fused q|k|v projection (active when dq > 0): columns [0, nq) are H query heads and
// [nq, nq + nk) KV key heads of dq dims each. Query and key heads are rotated on their pairs (p, p + dq/2) with
// the tables cos/sin [tables][HW][dq/2] of the row's board point (query head h uses its kv head's table; tables
// == 1 shares one; cos == nullptr: no rotation), and query columns are scaled by qscale.
struct QkvEpi {
  const float* cos = nullptr;
  const float* sin = nullptr;
  int dq = 0, nq = 0, nk = 0, H = 1, KV = 1, tables = 1;
  float qscale = 1.f;
};

struct GemmArgs {
  const void* A = nullptr; long lda = 0; long sA = 0;
  const void* Bt = nullptr; long ldb = 0; long sB = 0;
  long sC = 0;
  int M = 0, N = 0, K = 0, Z = 1;
  bool a_float = false;        // A holds float (converted, with `pro` applied when pro.scale)
  Prologue pro;
  ConvOut out;
  // Gated output (SwiGLU): the columns come in 16-wide pairs of blocks (value block, gate block) and the GEMM
  // writes only out.yt[m][f] = silu(C[m][32 (f / 16) + f % 16]) * C[m][32 (f / 16) + 16 + f % 16], f < N / 2.
  bool glu = false;
  // Activation of the compute-type output alone (ACT_ID or ACT_MISH): out.yt = act(C), as the mish FFN's h.
  int yt_act = ACT_ID;
  QkvEpi qkv;
  bool vec_epi = false;  // set by launch_gemm: the four-column vector epilogue applies
};
void launch_gemm(int prec, const GemmArgs& g, hipStream_t s);
// The rows of the row tile that launch_gemm runs a plain GEMM of these sizes on (row tile r on XCD r mod 8).
int gemm_row_tile(int prec, int M, int N, int K);

// Implicit-GEMM 1x1 / 3x3 "same" convolution on 16-bit operands: x compute-type NHWC rows of ldx (IC channels,
// IC % 8 == 0), w the compute-type conversion of conv_igemm_pack_weights' layout (icp = conv_igemm_icp(ks, IC)),
// OC % 4 == 0. Split (1x1 only): x_lo holds the low parts of the activation (Emit::out_lo, same layout) and w
// packs each output tile's high weight rows followed by their low parts; every product is then taken as
// hi*hi + lo*hi + hi*lo, which carries about 22 significant bits of each operand (a float-accurate convolution).
// Kernel-timing events for the next op (set by a profiled forward): every kernel launch (launch_k) then goes
// through hipExtLaunchKernel, whose dispatch records `start` before the op's first kernel and `stop` after each
// kernel, and sets `used`. An op that launches no kernel (a plain copy) is timed by events around it instead.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
  bool used = false;
};
extern thread_local LaunchTiming g_launch_timing;

int conv_igemm_icp(int ks, int ic, int oc, bool split = false);
// The profiling class of the configuration a convolution of these channel counts runs with (one per kernel
// instantiation: "conv3x3" is the 48-column 3x3 tile, "conv1x1_split_k128" the split 1x1 on 128-channel stages, ...).
const char* conv_igemm_class(int ks, int ic, int oc, bool split = false);
// Pixels per tile of the convolution of these channel counts (the tile of PoolPart's partials), and the columns
// per tile (BN) when its kernel computes pooling partials (3x3 with 64-channel column tiles, 192 pixels), else 0.
int conv_igemm_tile_rows(int ks, int ic, int oc, bool split = false);
int conv_igemm_pool_cols(int ks, int ic, int oc);
// The launch geometry of the convolution of these shapes over M pixels, and the index maps its kernel uses (the
// same functions): workgroup -> (pixel tile, column tile), -1 for a workgroup that exits at once; with the weights
// straight into LDS, the weight row and chunk that direct load q of (wave, lane) reads and the LDS row and chunk it
// fills (-1: the spare area), and the stored chunk of a row's logical chunk.
struct IgemmGeometry {
  int grid, threads, tile_rows, tile_cols, stage_channels, pixel_tiles, col_tiles, pairs;
  int weights_direct, weight_rows, waves, direct_instructions, direct_per_wave;
};
IgemmGeometry conv_igemm_geometry(int ks, int ic, int oc, bool split, int M);
void conv_igemm_tile_of(const IgemmGeometry& gm, int g, int& mt, int& nt);
void conv_igemm_weight_load(const IgemmGeometry& gm, int q, int wave, int lane, int& src_row, int& src_chunk,
                            int& dst_row, int& dst_chunk);
int conv_igemm_weight_chunk(int row, int chunk);
// w [oc][ic][ks][ks] -> [oc tile][tap][BN][icp] float; with `split` -> [oc tile][hi, lo][tap][BN][icp], the low
// plane holding w - round(w) for the compute type `prec`.
void conv_igemm_pack_weights(int ks, const float* w, int oc, int ic, std::vector<float>& out, bool split = false,
                             int prec = PREC_F16);
void launch_conv_igemm(int prec, int ks, const void* x, int ldx, int IC, const void* w, int icp, int OC,
                       const ConvOut& o, int B, hipStream_t s, const void* x_lo = nullptr);
// The value a float becomes as a compute-type operand (round to nearest even), as a float.
float conv_round_operand(float v, int prec);

// A nested-bottleneck junction in one launch (16-bit handles, split operands): block k's exit 1x1 convolution
// (kJunctionInner -> kJunctionOuter channels) into `exit_o` (the trunk's residual add, emitting the next block's
// activation), whose activation feeds block k + 1's entry 1x1 convolution (kJunctionOuter -> entry_oc, entry_oc
// kJunctionInner) into `entry_o` without passing through memory (exit_o.emit.out / out_lo are not written); or,
// after the trunk's last block, the heads' p1 | g1 | v1 convolution (entry_oc kJunctionHead, exit_o.y_dead: the
// trunk is read, not stored). x / x_lo: the exit's split operand (rows of ldx); w: the compute-type conversion of
// junction_pack_weights' layout of both filters (each [oc][ic]). The results equal the two separate split 1x1
// convolutions' bit for bit.
constexpr int kJunctionInner = 192, kJunctionOuter = 384, kJunctionHead = 96;
void junction_pack_weights(const float* w_exit, const float* w_entry, int entry_oc, int prec, std::vector<float>& out);
void launch_junction(int prec, const void* x, const void* x_lo, int ldx, const void* w, const ConvOut& exit_o,
                     const ConvOut& entry_o, int entry_oc, int B, hipStream_t s);
// The launch's grid over M pixels, and the 48-pixel tile workgroup g computes (tiles past M exit at once).
int junction_grid(int M);
// The stem junction: the network's stem, a 3x3 convolution of the packed input rows (ldx <= 32 channels, one 16-bit
// plane) into the trunk with its row bias (eo: y stored, colbias, the emission of the entry's activation), and the
// first nested block's entry 1x1 (384 -> 192, split operands), in one launch over junction_grid(M) workgroups.
// Weights: stem_junction_pack_weights of the stem's filters [384][ic][3][3] and the entry's [192][384].
void stem_junction_pack_weights(const float* w_stem, int ic, const float* w_entry, int entry_oc, int prec,
                                std::vector<float>& out);
void launch_stem_junction(int prec, const void* x, int ldx, const void* w, const ConvOut& eo, const ConvOut& no,
                          int B, hipStream_t s);
int junction_tile_of(int g);

// Network input planes, float NCHW [B][nin][361], to compute-type NHWC rows of ldo channels (zero beyond nin,
// ldo % 8 == 0), together with the board statistics of launch_mask_prep; with `gl.W` set, the same launch also
// computes the stem's per-row bias from the global inputs: out[b][o] = sum_i glob[b][i] * W[i][o] (W [nglob][C]).
struct InputGlobal {
  const float* glob = nullptr; int nglob = 0;
  const float* W = nullptr; int C = 0;
  float* out = nullptr;
};
void launch_input_prep(int prec, const float* bin, int nin, void* out, int ldo, float* mask, float* area, float* s1,
                       float* s2, int B, hipStream_t s, const InputGlobal& gl = InputGlobal());

// Direct odd-k "same" convolution, w as [ic][ky][kx][oc] float: x compute-type NHWC rows of ldx, or float NCHW.
void launch_conv_direct(int prec, const void* x, int ldx, bool nchw_f32, int IC, const float* w, int OC, int ky, int kx,
                        int dy, int dx, const ConvOut& o, int B, hipStream_t s);

// out[m][c] = T(act((x[m][c] + prebias[m / HW][c]) * scale[c] + bias[c]) * mask[m]) for c < C.
void launch_bias_act(int prec, const float* x, int ldx, int C, const float* prebias, int ld_prebias, const float* scale,
                     const float* bias, int act, const float* mask, void* out, int ldo, int rows, hipStream_t s);

// Zero `bytes` (a multiple of 4) at p, 16-byte aligned: a kernel rather than hipMemsetAsync, so that a caller may
// capture it in a graph.
void launch_fill_zero(void* p, size_t bytes, hipStream_t s);

// mask[b][pos] = bin[b][0][pos]; area = sum; s1 = (sqrt(area)-14)*0.1; s2 = (sqrt(area)-14)^2*0.01-0.1.
void launch_mask_prep(const float* bin, int nin, float* mask, float* area, float* s1, float* s2, int B,
                      hipStream_t s);

// Board pooling of channels [coff, coff+C) of x [B*HW][ldx] after the prologue:
// gpool (value=false): [mean, mean*s1, max(x + mask*1e4 - 1e4)]; value pool: [mean, mean*s1, mean*s2].
void launch_pool(const float* x, int ldx, int coff, int C, const Prologue& pro, const float* area,
                 const float* s1, const float* s2, bool value, float* out, int B, hipStream_t s);

// out[b][o*ostride] (+)= act(sum_i in[b][i] * W[i][o] + bias[o]).
void launch_small_matmul(const float* in, int ldin, int IC, const float* W, int OC, const float* bias, int act,
                         float* out, long ldout, int ostride, bool accumulate, int B, hipStream_t s);

// Per-row work of one batch row in one workgroup: up to two board poolings (as launch_pool) into LDS features, then
// up to eight small matmuls chained through LDS (out = act(in W + bias), written to LDS and/or to a global row with
// a stride, optionally accumulated). Replaces a pooling launch plus a launch per matmul.
struct RowPool {
  const float* x = nullptr; int ldx = 0, coff = 0, C = 0;
  // Or the producer's partials (PoolPart, tiles of ppt pixels): the row's sums and maxima are combined from them.
  const long long* psum = nullptr; const float* pmax = nullptr; int ppt = 0;
  const float* scale = nullptr; const float* bias = nullptr; int act = ACT_ID;  // prologue (scale null: none)
  bool value = false;
  int dst = 0;  // LDS float offset of the 3C features
};
struct RowMM {
  const float* gin = nullptr; int ldgin = 0;  // input row from global memory (row stride), else from LDS
  int src = 0;                                // LDS float offset of the input
  int IC = 0, OC = 0;
  const float* W = nullptr;                   // [IC][OC]
  const float* bias = nullptr; int act = ACT_ID;
  int dst = -1;                               // LDS float offset of the output, or -1
  float* out = nullptr; long ldout = 0; int ostride = 1; bool accumulate = false;
  int wlds = -1;                              // LDS float offset of a staged copy of W, or -1 (read from memory)
  int wcols = 0;                              // with wlds and output splits: the copy holds only this workgroup's
                                              // share of the columns, [IC][wcols]
  bool bias_lds = false;                      // with wlds (whole columns): the copy holds the bias after W, at
                                              // wlds + IC * OC (the bias follows W in memory too)
  int w4 = 0;                                 // 16-byte vectors in the staged copy (0 without wlds)
};
// Optional last stage: the workgroup's share [o0, o1) of the last matmul's outputs (kept in LDS at its dst) is a
// per-row channel bias, and out[m][c] = T(act((x[m][c] + bias_row[c]) * scale[c] + bias[c]) * mask[m]) for the
// row's HW points and c in [o0, o1) (launch_bias_act's arithmetic; 16-bit compute types only). Its loads of x are
// issued before the pooling, so they overlap it.
struct RowEmit {
  const float* x = nullptr; int ldx = 0;  // null: no emission
  const float* scale = nullptr; const float* bias = nullptr; int act = ACT_ID;
  void* out = nullptr; int ldo = 0; int prec = PREC_F16;
};
constexpr int RE_MAX = 4;  // emitted 8-channel vectors per thread: (o1 - o0) / 8 * HW <= RE_MAX * 1024
struct RowProg {
  RowPool pool[2]; int npool = 0;
  RowMM mm[8]; int nmm = 0;
  int lds_floats = 0;  // LDS features and intermediates
  int splits = 1;      // workgroups per row sharing the outputs of the (single) matmul
  const float* mask = nullptr; const float* area = nullptr; const float* s1 = nullptr; const float* s2 = nullptr;
  RowEmit emit;
};
// Whether a row program with `splits` output shares of an OC-output last matmul can carry an emission.
bool row_emit_fits(int OC, int splits);
// Independent row programs of one launch (blockIdx.y picks the program).
struct RowProgs {
  static constexpr int MAX = 3;
  RowProg p[MAX];
  int n = 0;
};
void launch_row_prog(const RowProg& p, int B, hipStream_t s);
void launch_row_progs(const RowProgs& ps, int B, hipStream_t s);
// A global-pooling block's mid activation per 192-pixel tile, with 16-bit compute types: workgroup (tile t, share
// s) runs on XCD t mod 8 (the XCD of the convolutions' tile t), and for each batch row b that the tile touches (at
// most two) combines the gpool branch's pooled features from the producer's partials (PoolPart, 192-pixel tiles:
// mean, mean * s1[b], max), multiplies them by W [3 cg][cr] for its `share` output channels (the row's per-channel
// bias), and emits out[m][c] = T(act((x[m][c] + bias_row[c]) * scale[c] + bias[c]) * mask[m]) for the tile's pixels
// and its channels. The matmul sums the same 16 K slices in the same order as the row program (run_row_prog with
// output splits), so both give the same bits. Then it touches the next op's weights into L2 (pf).
struct GpoolTile {
  const long long* psum = nullptr; const float* pmax = nullptr; int cg = 0;
  const float* area = nullptr; const float* s1 = nullptr;
  const float* W = nullptr; int cr = 0; int share = 0;
  const float* x = nullptr; int ldx = 0;
  const float* scale = nullptr; const float* bias = nullptr; int act = ACT_ID;
  const float* mask = nullptr;
  void* out = nullptr; int ldo = 0; int prec = PREC_F16;
  const char* pf = nullptr; int pf_bytes = 0;
};
// The output share launch_gpool_tile uses for cr channels (0: none fits: 64 <= 3 cg <= 384 and cr / 8 a multiple
// of 8 up to 40 are needed).
int gpool_tile_share(int cg, int cr);
// Its launch over M pixels with `shares` channel shares: 8 ceil(tiles / 8) shares workgroups; workgroup g takes
// tile (g mod 8) + 8 ((g / 8) / shares) (on XCD g mod 8, the convolutions' XCD of that tile) and share
// (g / 8) mod shares; tiles past the last pixel exit at once.
constexpr int kGpoolTileRows = 192;
inline int gpool_tile_grid(int M, int shares) { return 8 * ((M + kGpoolTileRows * 8 - 1) / (kGpoolTileRows * 8)) * shares; }
__host__ __device__ inline void gpool_tile_of(int g, int shares, int& tile, int& share) {
  const int j = g >> 3;
  tile = (g & 7) + 8 * (j / shares);
  share = j % shares;
}
void launch_gpool_tile(const GpoolTile& a, int B, hipStream_t s);

// Gives each matmul of `p` whose weights fit a staged copy in LDS (after the program's features), as long as the
// program's LDS stays within `max_bytes`.
void row_prog_stage_weights(RowProg& p, size_t max_bytes);

// Per board point: the policy conv p2 over act(BN(p1 + gpool bias)) * mask, and the ownership conv over
// act(BN(v1)) * mask, written into the readback rows.
struct HeadSpatialArgs {
  const float* H = nullptr; int ldh = 0;
  int p1_off = 0, c_p1 = 0; const float* p1_bias = nullptr;  // [B][c_p1]
  const float* p1_scale = nullptr; const float* p1_shift = nullptr; int p1_act = 0;
  const float* w_p2 = nullptr; int P = 0;                     // [c_p1][P]
  int v1_off = 0, c_v1 = 0;
  const float* v1_scale = nullptr; const float* v1_shift = nullptr; int v1_act = 0;
  const float* w_own = nullptr;                               // [c_v1]
  const float* mask = nullptr;
  float* out = nullptr; int row_len = 0; int own_off = 0;
};
void launch_head_spatial(const HeadSpatialArgs& a, int B, hipStream_t s);

// Copies n floats of device memory into pinned, coherent host memory with 16-byte stores over the bus, and makes
// them visible to the host before the kernel ends (a system-scope fence): the rows' readback as one kernel on the
// stream, without a DMA engine's start-up. Both pointers 16-byte aligned.
void launch_readback(const float* src, float* host_dst, size_t n, hipStream_t s);

// The first row of RMSNorm workgroup g when each takes per_wg consecutive rows: g per_wg, or (region > 0: the rows
// written in row tiles of `region` rows, tile r on XCD r mod 8, and region a multiple of per_wg) share `sub` of tile
// x + 8 k, x = g mod 8 being the workgroup's XCD.
__host__ __device__ inline int rmsnorm_first_row(int g, int region, int per_wg) {
  if (region <= 0) return g * per_wg;
  const int wpr = region / per_wg, slot = g >> 3, k = slot / wpr, sub = slot - k * wpr;
  return ((g & 7) + 8 * k) * region + sub * per_wg;
}
__host__ __device__ inline int rmsnorm_grid(int rows, int region, int per_wg) {
  return region > 0 ? 8 * ((rows + 8 * region - 1) / (8 * region)) * (region / per_wg) : (rows + per_wg - 1) / per_wg;
}
// Rows per workgroup of the vector RMSNorm kernel for rows of C channels (0: C takes the scalar kernel).
int rmsnorm_rows_per_workgroup(int C);

// Per-token RMSNorm of transformer blocks: out = x * (1/sqrt(sum(x^2)/C + eps)) * w * mask[row] (compute type).
// region > 0: x was written in row tiles of `region` rows, tile r on XCD r mod 8, and each workgroup takes its rows
// from a tile of its own XCD, so that they come from the L2 that holds them.
void launch_rmsnorm_tok(int prec, const float* x, int ldx, int C, const float* w, float eps, const float* mask,
                        void* out, int ldo, int rows, hipStream_t s, int region = 0);

// Trunk-tip RMSNorm: act(x * rms * gamma + beta) * mask, rms per point or over the board (spatial).
void launch_tip_rms(const float* x, int C, const float* gamma, const float* beta, float eps, bool spatial, int act,
                    const float* mask, const float* area, float* rs_tmp, float* out, int B, hipStream_t s);

// Softmax attention over the board on the fused projection buffer qkv [B*HW][ldq] (q | k | v columns), whose
// queries and keys carry RoPE already (the projection's epilogue, QkvEpi), queries times `scale`; key bias
// mask*3e4 - 3e4.
struct AttnArgs {
  const void* qkv = nullptr; int ldq = 0;
  int q_off = 0, k_off = 0, v_off = 0;
  int H = 0, KV = 0, dq = 0, dv = 0;
  float scale = 1.f;
  const float* mask = nullptr;
  void* out = nullptr; int ldo = 0;
};
void launch_attention(int prec, const AttnArgs& a, int B, hipStream_t s);

// The per-row output post-processing on the device (kgx_post.hip): copy_outputs (optimism mix, inverse symmetry,
// fields by model version) then NNEvaluator's policy softmax over the legal moves, value softmax, score transforms
// and tanh ownership. Output per row: POST_LEN floats, the policy probabilities [362] (-1 for illegal moves),
// then white win, loss, no-result probabilities, score mean, score mean square, lead, variance time left,
// short-term winloss and score errors [9], then the ownership [361] (white's perspective, 0 off the board).
// status[r]: 0, or bit 0 a nonfinite policy sum, bit 1 a nonfinite value or score field.
constexpr int POST_LEN = HW + 1 + 9 + HW;
struct PostRow {
  int symmetry = 0;          // 0..7 (bit 0 flips y, bit 1 flips x, bit 2 transposes)
  float optimism = 0.f;      // policy optimism
  int white_to_move = 0;     // the net's outputs are the player to move's: 1 when that is white
  int board_x = POS, board_y = POS;
  float policy_scale = 1.f;  // outputScaleMultiplier / nnPolicyTemperature
  int passing_hacks = 0;     // cap the pass prior at 19 times the other moves
  int no_result = 1;         // no-result outcomes count (simple ko or territory scoring)
};
struct PostModel {
  int P = 1, S = 6, version = 8;
  double pp[7] = {20, 20, 20, 20, 40, 0.25, 30};  // td score, score mean, score stdev, lead, variance time, st value
                                                   // error, st score error multipliers
};
void launch_post(const float* raw, int row_len, const PostRow* rows, const unsigned char* legal, const PostModel& m,
                 float* out, int* status, int n, hipStream_t s);

// The device featurizer (kgx_featurize.hip): rejects a position outside fill_row_v7's assumptions for an nn_x x nn_y
// layout; launches fill_row_v7 plus the input symmetry for n device-resident positions into n rows of 22 planes
// (NCHW, or NHWC) and n rows of ld_glob floats (the 19 globals first).
void validate_position(const kg_position& p, int nn_x, int nn_y);
void launch_featurize(const kg_position* rows, int n, int nn_x, int nn_y, bool nhwc, const int* syms, float* bin,
                      float* glob, int ld_glob, hipStream_t s);

// The static device workspace of the allocation-free forward pass (kg_run_static): its size, and its address on
// `device` (looked up once per device, with `device` current).
constexpr size_t kStaticScratchBytes = 64ull << 20;
void* static_scratch(int device);

// FFN activation: h = silu(u[:, :F]) * u[:, F:2F] (gated) or mish(u[:, :F]), u float [rows][ldu] -> compute type.
void launch_ffn_act(int prec, const float* u, int ldu, int F, bool gated, void* h, int ldh, int rows, hipStream_t s);

}  // namespace kgx
