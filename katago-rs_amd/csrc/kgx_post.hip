// The per-row output post-processing on the device: copy_outputs (crates/katago-nn-burn/src/backend.rs:622-731:
// policy optimism mix, inverse symmetry, value/score fields by model version) followed by NNEvaluator's
// arithmetic on the fields (crates/katago-core/src/neuralnet/nneval.rs:1197-1500: the policy softmax over the
// legal moves with its temperature and passing cap, the value softmax and score transforms by model version,
// and tanh ownership from white's perspective). The legality of each move (history.is_legal plus any dagger ban)
// is an input: it needs the rules engine, which stays with the caller.
//
// One workgroup of 384 threads per row: a thread per policy position (362) and per ownership point (361), a block
// reduction for the softmax's maximum, thread 0 for its sum (in position order) and for the scalar value and score
// fields, in double as the reference computes them. The arithmetic is the reference's operation by operation (this
// file is compiled without contraction into fused multiply-adds, as Rust does not contract), with glibc's expf and a
// correctly rounded tanhf, so that the results equal the reference's bit for bit.
#include "kgx_device.h"
#include "kgx_expf.h"

#include <cmath>

namespace kgx {

namespace {

constexpr int PNT = 384;         // threads per row
constexpr int NPOL = HW + 1;     // policy positions, pass last

// Index of source point (h, w) of the 19x19 grid in the destination of copy_outputs' symmetry (reverse =
// true: nninputs.rs:877-879 copy_outputs_with_symmetry; bit 0 flips y, bit 1 flips x, bit 2 transposes).
__device__ __forceinline__ int sym_dst(int h, int w, int sym) {
  const bool tr = (sym & 4) != 0, fx = (sym & 2) != 0, fy = (sym & 1) != 0;
  int hb = 0, hs = POS, wb = 0, ws = 1;
  if (fy) { hb = (POS - 1) * POS; hs = -POS; }
  if (fx) { wb = POS - 1; ws = -1; }
  if (tr) { const int t = hs; hs = ws; ws = t; }
  return hb + h * hs + wb + w * ws;
}

__device__ __forceinline__ double soft_plus(double x) { return x > 40.0 ? x : log(1.0 + exp(x)); }

// expf as glibc computes it (the reference calls its port of glibc's, crates/katago-core/src/port/math.rs:634-680,
// so the policy probabilities match bit for bit): exp(x) = 2^(k/32) 2^(r/32) with x 32/ln 2 = k + r, r in [-1/2, 1/2]
// (found with fused multiply-adds in double), 2^(k/32) from a table and 2^(r/32) from a cubic (kgx_expf.h), then one
// rounding to float. Below log(2^-150) the result is 0, up to log(2^-149) the least subnormal, as glibc's underflow
// paths return. tests/expf_check.cpp checks the same steps and constants against the host's glibc expf.
__device__ float expf_glibc(float x) {
  const unsigned u = __float_as_uint(x), abstop = (u >> 20) & 0x7ff;
  if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88, or x is not finite
    if (u == 0xff800000u) return 0.f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > __uint_as_float(0x42b17217u)) return __uint_as_float(0x7f800000u);
    if (x < __uint_as_float(0xc2cff1b4u)) return 0.f;
    if (x < __uint_as_float(0xc2ce8ecfu)) return __uint_as_float(1u);
  }
  const double xd = (double)x;
  double kd = __builtin_fma(kgx_exp2f_invln2n, xd, kgx_exp2f_shift);
  const unsigned long long ki = (unsigned long long)__double_as_longlong(kd);
  kd -= kgx_exp2f_shift;
  const double r = __builtin_fma(kgx_exp2f_invln2n, xd, -kd);
  const double sc = __longlong_as_double((long long)(kgx_exp2f_tab[ki % 32] + (ki << 47)));
  const double z = __builtin_fma(kgx_exp2f_c0, r, kgx_exp2f_c1);
  const double r2 = r * r;
  double y = __builtin_fma(kgx_exp2f_c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y *= sc;
  return (float)y;
}

// tanhf correctly rounded, as the reference's (port/math.rs:804-853, glibc 2.44's): the double tanh rounded to
// float. It differs from the correct rounding only where the double's own error (an ulp or two of a double) straddles
// a float rounding boundary, about one value in 2^27.
__device__ float tanhf_cr(float x) {
  const float ax = fabsf(x);
  if (!(ax >= 0x1p-13f && ax < 10.0f)) {
    if (x != x) return x + x;
    if (ax < 0x1p-13f) return x;  // tanh(x) = x - x^3/3 + ... rounds to x
    return x > 0.f ? 1.f : -1.f;   // 1 - tanh(x) < 2^-27: rounds to 1
  }
  const float t = (float)tanh((double)ax);
  return x > 0.f ? t : -t;
}

// Block reductions over the 6 waves.
__device__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
  for (int k = 1; k < PNT / 64; k++) m = fmaxf(m, red[k]);
  return m;
}
__device__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int k = 0; k < PNT / 64; k++) s += red[k];
  return s;
}

__global__ __launch_bounds__(PNT) void post_kernel(const float* __restrict__ raw, int row_len,
                                                   const PostRow* __restrict__ rows,
                                                   const unsigned char* __restrict__ legal, PostModel m,
                                                   float* __restrict__ out, int* __restrict__ status) {
  const int r = blockIdx.x, t = threadIdx.x;
  const PostRow pr = rows[r];
  const float* row = raw + (size_t)r * row_len;
  const float* own_raw = row + m.P * NPOL + 3 + m.S;
  __shared__ float pol[NPOL], own[HW], red[PNT / 64 + NPOL + 2];  // (red: the block reductions, then the numerators)

  // copy_outputs: the optimism mix of the first two policy channels (P = 2, or P = 4 from version 16) and the
  // inverse symmetry of the policy's board part and of the ownership.
  const bool mix = m.P == 2 || (m.P == 4 && m.version >= 16);
  if (t < NPOL) {
    float p = row[t];
    if (mix) {
      const float po = row[NPOL + t];
      p = p + (po - p) * pr.optimism;
    }
    if (t < HW) {
      const int d = sym_dst(t / POS, t % POS, pr.symmetry);
      pol[d] = p;
      own[d] = own_raw[t];
    } else {
      pol[HW] = p;
    }
  }
  __syncthreads();

  // NNEvaluator's policy: illegal moves at -1e30, the others scaled by outputScaleMultiplier / temperature; the
  // softmax over all positions; optionally the pass prior capped at 19x the other moves' sum (floored at 1e-20);
  // legal moves get p / sum (or 1 / #legal when everything rounded to 0), the others -1.
  // The maximum starts at -1e25 and the sum is taken in position order by one thread, as the reference's loops
  // (nneval.rs:1235-1262), so that every probability is the reference's to the bit.
  const bool lg = t < NPOL && legal[(size_t)r * NPOL + t] != 0;
  const float v = t < NPOL ? (lg ? pol[t] * pr.policy_scale : -1e30f) : -INFINITY;
  const float mx = fmaxf(-1e25f, block_max(v, red));
  const float nlegal = block_sum(lg ? 1.f : 0.f, red);
  float e = t < NPOL ? expf_glibc(v - mx) : 0.f;
  float* const es = red + PNT / 64;  // [NPOL] the numerators, then [1] the sum
  if (t < NPOL) es[t] = e;
  __syncthreads();
  if (t == 0) {
    float s = 0.f;
    for (int i = 0; i < HW; i++) s += es[i];
    float ep = es[HW];
    if (pr.passing_hacks) ep = fmaxf(1e-20f, fminf(ep, s * 19.f));
    es[NPOL] = ep;
    es[NPOL + 1] = s + ep;
  }
  __syncthreads();
  if (t == HW) e = es[NPOL];
  const float sum = es[NPOL + 1];
  float* o = out + (size_t)r * POST_LEN;
  if (t < NPOL) {
    float p;
    if (!lg) p = -1.f;
    else if (sum <= 0.f) p = 1.f / nlegal;
    else p = e / sum;
    o[t] = p;
  }
  int st = isfinite(sum) ? 0 : 1;

  // Ownership from white's perspective, 0 off the board.
  if (t < HW) {
    const int y = t / POS, x = t % POS;
    float w = 0.f;
    if (y < pr.board_y && x < pr.board_x) {
      const float th = tanhf_cr(own[t]);
      w = pr.white_to_move ? th : -th;
    }
    o[NPOL + 9 + t] = w;
  }

  // Value and score fields (thread 0), in double.
  if (t == 0) {
    const float* val = row + m.P * NPOL;
    const float* sc = val + 3;
    // copy_outputs' fields by model version.
    float f_mean, f_mean_sq, f_lead, f_var, f_stw, f_sts;
    if (m.version >= 9) {
      f_mean = sc[0]; f_mean_sq = sc[1]; f_lead = sc[2]; f_var = sc[3]; f_stw = sc[4]; f_sts = sc[5];
    } else if (m.version >= 8) {
      f_mean = sc[0]; f_mean_sq = sc[1]; f_lead = sc[2]; f_var = sc[3]; f_stw = 0.f; f_sts = 0.f;
    } else if (m.version >= 4) {
      f_mean = sc[0]; f_mean_sq = sc[1]; f_lead = f_mean; f_var = 0.f; f_stw = 0.f; f_sts = 0.f;
    } else {
      f_mean = sc[0]; f_mean_sq = f_mean * f_mean; f_lead = f_mean; f_var = 0.f; f_stw = 0.f; f_sts = 0.f;
    }
    const bool white = pr.white_to_move != 0;
    const double win_l = (double)val[0], loss_l = (double)val[1];
    double nores_l = (double)val[2];
    float res[9];
    if (m.version == 3) {
      // The pre-arctanned score value: atanf of the float (the float overload), times 2 / pi.
      const double two_over_pi = 0.63661977236758134308;
      const double score_value = (double)atanf(f_mean) * two_over_pi;
      const double mxl = fmax(fmax(win_l, loss_l), nores_l);
      double wp = exp(win_l - mxl), lp = exp(loss_l - mxl), np = exp(nores_l - mxl);
      const double ps = wp + lp + np;
      wp /= ps; lp /= ps; np /= ps;
      if (!isfinite(ps) || !isfinite(score_value)) st |= 2;
      // approx_white_score_of_score_value_smooth(scoreValue, 0, 2, sqrt(board area)): tan(v pi / 2), clamped.
      const double half_pi = 1.57079632679489661923, x = score_value * half_pi;
      const double unscaled = x >= half_pi - 1e-6 ? 1e6 : x <= -half_pi + 1e-6 ? -1e6 : tan(x);
      const float smean = (float)(unscaled * (2.0 * sqrt((double)pr.board_x * (double)pr.board_y)));
      const float wmean = white ? smean : -smean;
      res[0] = (float)(white ? wp : lp); res[1] = (float)(white ? lp : wp); res[2] = (float)np;
      res[3] = wmean; res[4] = wmean * wmean; res[5] = wmean;
      res[6] = -1.f; res[7] = -1.f; res[8] = -1.f;
    } else {
      if (!pr.no_result) nores_l -= 100000.0;
      const double mxl = fmax(fmax(win_l, loss_l), nores_l);
      double wp = exp(win_l - mxl), lp = exp(loss_l - mxl), np = exp(nores_l - mxl);
      if (!pr.no_result) np = 0.0;
      const double ps = wp + lp + np;
      wp /= ps; lp /= ps; np /= ps;
      double mean = (double)f_mean * m.pp[1];
      const double stdev = soft_plus((double)f_mean_sq) * m.pp[2];
      double mean_sq = mean * mean + stdev * stdev;
      double lead = (double)f_lead * m.pp[3];
      const double var = soft_plus((double)f_var) * m.pp[4];
      mean *= 1.0 - np;
      mean_sq *= 1.0 - np;
      lead *= 1.0 - np;
      double stw, sts;
      if (m.version >= 14) {
        const double a = soft_plus((double)f_stw * 0.5), b = soft_plus((double)f_sts * 0.5);
        stw = sqrt(a * a * m.pp[5]);
        sts = sqrt(b * b * m.pp[6]);
      } else if (m.version >= 10) {
        stw = sqrt(soft_plus((double)f_stw) * m.pp[5]);
        sts = sqrt(soft_plus((double)f_sts) * m.pp[6]);
      } else {
        stw = soft_plus((double)f_stw);
        sts = soft_plus((double)f_sts) * 10.0;
      }
      if (!isfinite(ps) || !isfinite(mean) || !isfinite(mean_sq) || !isfinite(lead) || !isfinite(var) ||
          !isfinite(stw) || !isfinite(sts))
        st |= 2;
      res[0] = (float)(white ? wp : lp); res[1] = (float)(white ? lp : wp); res[2] = (float)np;
      res[3] = white ? (float)mean : -(float)mean;
      res[4] = (float)mean_sq;
      res[5] = white ? (float)lead : -(float)lead;
      if (m.version >= 9) {
        res[6] = (float)var; res[7] = (float)stw; res[8] = (float)sts;
      } else {
        res[6] = -1.f; res[7] = -1.f; res[8] = -1.f;
      }
    }
    for (int k = 0; k < 9; k++) o[NPOL + k] = res[k];
    status[r] = st;
  }
}

}  // namespace

void launch_post(const float* raw, int row_len, const PostRow* rows, const unsigned char* legal, const PostModel& m,
                 float* out, int* status, int n, hipStream_t s) {
  if (n <= 0) return;
  if (m.version < 3) throw std::runtime_error("NNEval value postprocessing not implemented for model version");
  launch_k(post_kernel, dim3(n), dim3(PNT), 0, s, raw, row_len, rows, legal, m, out, status);
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
