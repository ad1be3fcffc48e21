// The device featurizer: NNInputs::fill_row_v7 (crates/katago-core/src/neuralnet/nninputs.rs:1336-1800) for positions
// given by their board and the rules engine's results (kg_position), followed by copy_inputs' symmetry
// (crates/katago-nn-burn/src/backend.rs:497-546, nninputs.rs:756-874), writing the rows a forward pass reads.
//
// One workgroup per position, one thread per point. The board's chains are labelled in LDS by repeated minimum
// propagation between same-coloured neighbours (with a jump to the label's own label), double-buffered so that a
// step reads only the previous step's labels; a chain's label is then its smallest point. Every empty point adds
// one liberty to each distinct chain next to it (LDS atomics), which is Board::get_num_liberties: the number of
// distinct empty points next to the chain. Each thread then writes the 22 features of its point at the point's
// symmetric position; thread 0 writes the 19 global features.
#include "kgx_device.h"

namespace kgx {

namespace {

constexpr int FEAT = 22, GLOB = 19, FT = 384;  // features, globals, threads per workgroup (>= 361 points)

// The destination of source point (y, x) of an h x w plane under copy_inputs_with_symmetry (nninputs.rs:756-850):
// bit 2 transposes (square planes only; for inputs a transpose swaps the two flips), bit 1 flips x, bit 0 flips y.
__host__ __device__ inline int sym_dest(int y, int x, int h, int w, int sym) {
  const bool tr = (sym & 4) && h == w;
  bool fx = (sym & 2) != 0, fy = (sym & 1) != 0;
  if (tr) {
    const bool t = fx;
    fx = fy;
    fy = t;
  }
  const int r = tr ? x : y, c = tr ? y : x;
  return (fy ? h - 1 - r : r) * w + (fx ? w - 1 - c : c);
}

__global__ __launch_bounds__(FT) void featurize_kernel(const kg_position* __restrict__ rows, int nn_x, int nn_y,
                                                        int nhwc, const int* __restrict__ syms, float* __restrict__ bin,
                                                        float* __restrict__ glob, int ld_glob) {
  const int r = blockIdx.x, t = threadIdx.x;
  const kg_position& P = rows[r];
  __shared__ unsigned char col[HW];
  __shared__ int lab[2][HW];
  __shared__ int lib[HW];
  const int xs = P.x_size, ys = P.y_size, n = xs * ys, pla = P.next_player, opp = 3 - pla;
  const int x = t % xs, y = t / xs;
  if (t < n) col[t] = P.color[t];
  if (t < HW) lib[t] = 0;
  __syncthreads();
  const bool stone = t < n && col[t] != 0;
  if (t < n) lab[0][t] = stone ? t : -1;
  __syncthreads();
  // Chain labels: at most one step per point of the longest chain, each a workgroup-wide pass.
  int cur = 0;
  for (int it = 0; it < n; it++) {
    bool changed = false;
    if (stone) {
      const int* L = lab[cur];
      const unsigned char c = col[t];
      int m = L[t];
      if (x > 0 && col[t - 1] == c) m = min(m, L[t - 1]);
      if (x + 1 < xs && col[t + 1] == c) m = min(m, L[t + 1]);
      if (y > 0 && col[t - xs] == c) m = min(m, L[t - xs]);
      if (y + 1 < ys && col[t + xs] == c) m = min(m, L[t + xs]);
      m = min(m, L[m]);
      changed = m != L[t];
      lab[cur ^ 1][t] = m;
    }
    cur ^= 1;
    if (!__syncthreads_or(changed)) break;
  }
  const int* L = lab[cur];
  // Liberties: each empty point counts once for each distinct chain next to it.
  if (t < n && col[t] == 0) {
    int seen[4], k = 0;
    const int nb[4] = {x > 0 ? t - 1 : -1, x + 1 < xs ? t + 1 : -1, y > 0 ? t - xs : -1, y + 1 < ys ? t + xs : -1};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int q = nb[j];
      if (q < 0 || col[q] == 0) continue;
      const int l = L[q];
      bool dup = false;
      for (int i = 0; i < k; i++) dup |= seen[i] == l;
      if (!dup) {
        seen[k++] = l;
        atomicAdd(&lib[l], 1);
      }
    }
  }
  __syncthreads();

  // History: the most recent moves while they alternate opp, pla, opp, ...
  const int hmax = min(min(P.history_turns, P.num_moves), 5);
  int turns = 0;
  while (turns < hmax && P.move_player[turns] == ((turns & 1) ? pla : opp)) turns++;
  const int np = nn_x * nn_y, enc_phase = P.encore_phase;
  const bool has_area = P.scoring_rule == 0 || enc_phase >= 2;
  const int sym = syms ? syms[r] : 0;
  if (t < np) {
    const int gx = t % nn_x, gy = t / nn_x;
    float v[FEAT];
#pragma unroll
    for (int f = 0; f < FEAT; f++) v[f] = 0.f;
    if (gx < xs && gy < ys) {
      const int p = gx + gy * xs;
      const int c = col[p], mk = P.marks[p], a = P.area[p], e = P.encore_start[p];
      v[0] = 1.f;
      v[1] = c == pla;
      v[2] = c == opp;
      if (c) {
        const int l = lib[L[p]];
        v[3] = l == 1;
        v[4] = l == 2;
        v[5] = l == 3;
      }
      if (enc_phase == 0) {
        v[6] = p == P.ko_loc || (mk & 1);
      } else {
        v[6] = mk & 1;
        v[7] = (mk >> 1) & 1;
      }
      for (int k = 0; k < turns; k++)
        if (P.move_loc[k] == p) v[9 + k] = 1.f;
#pragma unroll
      for (int b = 0; b < 4; b++) v[14 + b] = (mk >> (2 + b)) & 1;
      if (has_area) {
        if (a == pla) v[18] = 1.f;
        else if (a == opp) v[19] = 1.f;
        else if (P.scoring_rule == 1) {
          if (c == pla && e == pla) v[18] = 1.f;
          else if (c == opp && e == opp) v[19] = 1.f;
        }
      }
      if (enc_phase >= 2) {
        v[20] = e == pla;
        v[21] = e == opp;
      }
    }
    const int d = sym_dest(gy, gx, nn_y, nn_x, sym);
    float* row = bin + (size_t)r * FEAT * np;
    if (nhwc) {
#pragma unroll
      for (int f = 0; f < FEAT; f++) row[(size_t)d * FEAT + f] = v[f];
    } else {
#pragma unroll
      for (int f = 0; f < FEAT; f++) row[(size_t)f * np + d] = v[f];
    }
  }

  if (t == 0) {
    float g[GLOB];
    for (int i = 0; i < GLOB; i++) g[i] = 0.f;
    for (int k = 0; k < turns; k++)
      if (P.move_loc[k] == -1) g[k] = 1.f;
    // Komi, bounded by the board area plus 20 (NNPos::KOMI_CLIP_RADIUS), over 20.
    float komi = P.self_komi;
    const float b_area = (float)n;
    if (komi > b_area + 20.0f) komi = b_area + 20.0f;
    if (komi < -b_area - 20.0f) komi = -b_area - 20.0f;
    g[5] = komi / 20.0f;
    if (P.ko_rule == 1 || P.ko_rule == 3) {
      g[6] = 1.f;
      g[7] = 0.5f;
    } else if (P.ko_rule == 2) {
      g[6] = 1.f;
      g[7] = -0.5f;
    }
    if (P.multi_stone_suicide_legal) g[8] = 1.f;
    if (P.scoring_rule == 1) g[9] = 1.f;
    if (P.tax_rule == 1) g[10] = 1.f;
    if (P.tax_rule == 2) {
      g[10] = 1.f;
      g[11] = 1.f;
    }
    if (enc_phase > 0) g[12] = 1.f;
    if (enc_phase > 1) g[13] = 1.f;
    g[14] = P.pass_would_end_phase ? 1.f : 0.f;
    if (P.playout_doubling_advantage != 0.0) {
      g[15] = 1.f;
      g[16] = (float)(0.5 * P.playout_doubling_advantage);
    }
    if (P.has_button) g[17] = 1.f;
    if (has_area) {
      // The komi parity wave: a triangle wave of period 2 around the komis that allow a draw (area parity).
      const float fl = (n % 2 == 0) ? floorf(komi / 2.0f) * 2.0f : floorf((komi - 1.0f) / 2.0f) * 2.0f + 1.0f;
      float dl = komi - fl;
      dl = dl < 0.f ? 0.f : dl > 2.f ? 2.f : dl;
      g[18] = dl < 0.5f ? dl : dl < 1.5f ? 1.0f - dl : dl - 2.0f;
    }
    for (int i = 0; i < GLOB; i++) glob[(size_t)r * ld_glob + i] = g[i];
  }
}

}  // namespace

// The reference asserts these (debug_assert / unreachable! in fill_row_v7 and the rules): a position outside them
// is rejected before any launch.
void validate_position(const kg_position& p, int nn_x, int nn_y) {
  auto bad = [](const std::string& m) { throw std::runtime_error("kgx featurizer: " + m); };
  if (p.x_size < 1 || p.y_size < 1 || p.x_size > nn_x || p.y_size > nn_y)
    bad("board size " + std::to_string(p.x_size) + "x" + std::to_string(p.y_size) + " outside the " +
        std::to_string(nn_x) + "x" + std::to_string(nn_y) + " layout");
  const int n = p.x_size * p.y_size;
  if (p.next_player != 1 && p.next_player != 2) bad("next_player must be 1 (black) or 2 (white)");
  if (p.ko_loc < -1 || p.ko_loc >= n) bad("ko_loc off the board");
  if (p.encore_phase < 0 || p.encore_phase > 2) bad("encore_phase must be 0, 1 or 2");
  if (p.ko_rule < 0 || p.ko_rule > 3 || p.scoring_rule < 0 || p.scoring_rule > 1 || p.tax_rule < 0 || p.tax_rule > 2)
    bad("unknown rules");
  if (p.num_moves < 0 || p.num_moves > 5 || p.history_turns < 0) bad("bad move history");
  for (int k = 0; k < p.num_moves; k++)
    if (p.move_loc[k] < -2 || p.move_loc[k] >= n || p.move_player[k] < 0 || p.move_player[k] > 2)
      bad("bad move history");
  for (int i = 0; i < n; i++)
    if (p.color[i] > 2 || p.area[i] > 2 || p.encore_start[i] > 2 || p.marks[i] > 63) bad("bad point value");
}

void launch_featurize(const kg_position* rows, int n, int nn_x, int nn_y, bool nhwc, const int* syms, float* bin,
                      float* glob, int ld_glob, hipStream_t s) {
  if (n <= 0) return;
  if (nn_x < 1 || nn_y < 1 || nn_x * nn_y > HW) throw std::runtime_error("kgx featurizer: layout larger than 19x19");
  launch_k(featurize_kernel, dim3(n), FT, 0, s, rows, nn_x, nn_y, nhwc ? 1 : 0, syms, bin, glob, ld_glob);
  KGX_CHECK_LAUNCH();
}

}  // namespace kgx
