// The C ABI (include/kgx.h): model loading, handles, the forward pass, and get_output with the reference's
// input and output handling (crates/katago-nn-burn/src/backend.rs:410-731).
#include "kgx.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "kgx_model.h"
#include "kgx_net.h"

struct kg_net {
  std::shared_ptr<const kgx::ModelDesc> model;  // shared with the handles, which may outlive the net object
};

struct kg_handle {
  int device = 0;
  int max_batch = 0;
  int precision = 0;
  hipStream_t stream = nullptr;
  std::unique_ptr<kgx::Net> net;
  // The model (kept for the allocation-free plan), and the plan of kg_run_static with its workspace in the static
  // scratch, made by its first call on the handle: static_batch is -1 before, then the plan's largest batch (0 when
  // one row's workspace does not fit).
  std::shared_ptr<const kgx::ModelDesc> model;
  std::unique_ptr<kgx::Net> net_static;
  int static_batch = -1;
  std::vector<int> buckets;
  int model_version = 0, P = 1, S = 1, nin = 0, nglob = 0, nmeta = 0;
  // Pinned host staging: the InputBuffers of the reference (backend.rs:150-212) and the readback.
  float* h_bin = nullptr;
  float* h_glob = nullptr;
  float* h_meta = nullptr;
  float* h_out = nullptr;
  // Buffers of the device post-processing (kg_get_output_eval, kg_post_outputs), allocated by their first call:
  // device raw rows (kg_post_outputs' input), per-row parameters, legality, outputs and status, with pinned host
  // staging for all but the raw rows (staged through h_out).
  float* d_post_raw = nullptr;
  kgx::PostRow* d_post_rows = nullptr;
  unsigned char* d_legal = nullptr;
  float* d_post_out = nullptr;
  int* d_post_status = nullptr;
  kgx::PostRow* h_post_rows = nullptr;
  unsigned char* h_legal = nullptr;
  float* h_post_out = nullptr;
  int* h_post_status = nullptr;
  kgx::PostModel post_model;
  // The device featurizer's staging (kg_featurize, first use): one pinned block of the symmetries (max_batch ints,
  // padded to 256 bytes) followed by the positions, which the kernel reads over the bus (no copy of its own); and an
  // event after that kernel (the next call waits for it before overwriting the staging).
  char* h_feat = nullptr;
  size_t feat_sym_bytes = 0;
  hipEvent_t pos_uploaded = nullptr;
  bool pos_pending = false;
  // The readback of kg_get_output_async runs on this helper thread; the next call on the handle joins it first.
  std::thread helper;
  int helper_status = 0;
  std::string helper_error;
  std::mutex mu;
};

namespace {

thread_local std::string g_last_error;

int fail(const std::string& msg) {
  g_last_error = msg;
  return 1;
}

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    return fail(e.what());
  }
}

constexpr int POS = 19;
constexpr int HW = POS * POS;

// copyWithSymmetry (crates/katago-core/src/neuralnet/nninputs.rs:756-850), NCHW, one row: flipY = bit 0,
// flipX = bit 1, transpose = bit 2 on square boards; for inputs (reverse = false) a transpose swaps the flips.
// The destination offset walks h_base + h * h_stride + w_base + w * w_stride with the strides exchanged by a
// transpose, exactly as the reference.
void copy_with_symmetry(const float* src, float* dst, int c_size, int h_size, int w_size, int symmetry, bool reverse) {
  const bool transpose = (symmetry & 0x4) != 0 && h_size == w_size;
  bool flip_x = (symmetry & 0x2) != 0;
  bool flip_y = (symmetry & 0x1) != 0;
  if (transpose && !reverse) std::swap(flip_x, flip_y);
  const int nc_stride = h_size * w_size;
  int h_base = 0, h_stride = w_size, w_base = 0, w_stride = 1;
  if (flip_y) {
    h_base = (h_size - 1) * h_stride;
    h_stride = -h_stride;
  }
  if (flip_x) {
    w_base = (w_size - 1) * w_stride;
    w_stride = -w_stride;
  }
  if (transpose) std::swap(h_stride, w_stride);
  for (int nc = 0; nc < c_size; nc++) {
    const float* s = src + (size_t)nc * nc_stride;
    float* d = dst + (size_t)nc * nc_stride;
    for (int h = 0; h < h_size; h++)
      for (int w = 0; w < w_size; w++) d[h_base + h * h_stride + w_base + w * w_stride] = s[h * w_size + w];
  }
}

// NNModelVersion's input layout per model version (crates/katago-core/src/neuralnet/modelversion.rs:40-110):
// the inputs version, spatial and global feature counts; versions outside 3..17 fail with the reference's text.
void model_version_features(int v, int& inputs_version, int& spatial, int& global) {
  if (v < 3 || v > 17)
    throw std::runtime_error("NNModelVersion: Model version not currently implemented or supported: " + std::to_string(v));
  static const int iv[5] = {3, 4, 5, 6, 7}, sp[5] = {22, 22, 13, 22, 22}, gl[5] = {14, 14, 12, 16, 19};
  const int k = v <= 4 ? 0 : v >= 8 ? 4 : v - 4;  // inputs versions 3 (v3-4), 4 (v5), 5 (v6), 6 (v7), 7 (v8+)
  inputs_version = iv[k];
  spatial = sp[k];
  global = gl[k];
}

// NNModelVersion::getNumInputMetaChannels (modelversion.rs): 0 without an SGF metadata encoder, 192 with one.
int meta_encoder_channels(int meta_version) {
  if (meta_version == 0) return 0;
  if (meta_version == 1) return 192;
  throw std::runtime_error("NNModelVersion: metaEncoderVersion not currently implemented or supported: " +
                           std::to_string(meta_version));
}

// copy_outputs (crates/katago-nn-burn/src/backend.rs:622-731): one readback row of P*362 + 3 + S + 361 floats to
// NNOutput fields. The policy mixes channel 1 (optimistic) into channel 0 by the row's optimism for P == 2 or for
// P == 4 from model version 16; policy and ownership are mapped back through the row's symmetry; the score fields
// are unpacked by model version.
void copy_outputs_row(const float* row, int P, int S, int v, int sym, float optimism, kg_nn_output& o) {
  float tmp[HW];
  const float* pol = row;
  if (P == 2 || (P == 4 && v >= 16)) {
    for (int i = 0; i < HW; i++) {
      const float p = pol[i], po = pol[(HW + 1) + i];
      tmp[i] = p + (po - p) * optimism;
    }
    copy_with_symmetry(tmp, o.policy_probs, 1, POS, POS, sym, true);
    const float p0 = pol[HW], p1 = pol[(HW + 1) + HW];
    o.policy_probs[HW] = p0 + (p1 - p0) * optimism;
  } else {
    copy_with_symmetry(pol, o.policy_probs, 1, POS, POS, sym, true);
    o.policy_probs[HW] = pol[HW];
  }
  const float* val = row + P * (HW + 1);
  const float* sc = val + 3;
  const float* own = sc + S;
  o.white_win_prob = val[0];
  o.white_loss_prob = val[1];
  o.white_no_result_prob = val[2];
  if (o.white_owner_map) copy_with_symmetry(own, o.white_owner_map, 1, POS, POS, sym, true);
  if (v >= 9) {
    o.white_score_mean = sc[0]; o.white_score_mean_sq = sc[1]; o.white_lead = sc[2]; o.var_time_left = sc[3];
    o.shortterm_winloss_error = sc[4]; o.shortterm_score_error = sc[5];
  } else if (v >= 8) {
    o.white_score_mean = sc[0]; o.white_score_mean_sq = sc[1]; o.white_lead = sc[2]; o.var_time_left = sc[3];
    o.shortterm_winloss_error = 0.f; o.shortterm_score_error = 0.f;
  } else if (v >= 4) {
    o.white_score_mean = sc[0]; o.white_score_mean_sq = sc[1]; o.white_lead = o.white_score_mean;
    o.var_time_left = 0.f; o.shortterm_winloss_error = 0.f; o.shortterm_score_error = 0.f;
  } else {
    // Version 3 nets have no second moment output: the mean squared stands in for it.
    o.white_score_mean = sc[0]; o.white_score_mean_sq = o.white_score_mean * o.white_score_mean;
    o.white_lead = o.white_score_mean; o.var_time_left = 0.f; o.shortterm_winloss_error = 0.f;
    o.shortterm_score_error = 0.f;
  }
}

// The score-value channel count each model version's value head has (bin2onnx.py:849-856).
int score_channels_for_version(int v) { return v >= 9 ? 6 : v >= 8 ? 4 : v >= 4 ? 2 : 1; }

int padded_batch_size(const std::vector<int>& buckets, int n, int max_batch) {
  int best = -1;
  for (int b : buckets)
    if (b >= n && b <= max_batch && (best < 0 || b < best)) best = b;
  return best < 0 ? n : best;
}

// Plans kg_run_static's forward pass in the device's static scratch, for the largest batch up to max_batch whose
// workspace fits (the workspace grows linearly with the batch, up to tile rounding). Planning allocates no device
// memory; it looks up the scratch's address on the handle's device (once per device), reuses the handle's weights
// and assigns workspace addresses.
void plan_static(kg_handle* h, const kgx::ModelDesc& m) {
  char* base = (char*)kgx::static_scratch(h->device);
  const size_t cap = kgx::kStaticScratchBytes;
  auto plan = std::make_unique<kgx::Net>(m, *h->net, h->max_batch, base, cap);
  int b = h->max_batch;
  if (!plan->fits()) {
    const size_t wmax = plan->workspace_bytes();
    auto one = std::make_unique<kgx::Net>(m, *h->net, 1, base, cap);
    plan.reset();
    b = 0;
    if (one->fits()) {
      const double per_row = (double)(wmax - one->workspace_bytes()) / (h->max_batch - 1);
      b = std::min(h->max_batch - 1, 1 + (int)((double)(cap - one->workspace_bytes()) / per_row));
      for (; b > 1; b--) {
        plan = std::make_unique<kgx::Net>(m, *h->net, b, base, cap);
        if (plan->fits()) break;
        plan.reset();
      }
      if (b == 1) plan = std::move(one);
    }
  }
  h->static_batch = plan ? b : 0;
  h->net_static = std::move(plan);
}

// Runs the first `n_run` rows already staged in the device input buffers; reads `n` rows back into h_out.
void run_and_read(kg_handle* h, int n_run, int n, float* out) {
  h->net->forward(n_run, h->stream);
  const size_t bytes = (size_t)n * h->net->row_len() * sizeof(float);
  kgx::launch_readback(h->net->d_out(), h->h_out, bytes / sizeof(float), h->stream);
  KGX_HIP(hipStreamSynchronize(h->stream));
  if (out) std::memcpy(out, h->h_out, bytes);
}

// Joins the helper thread of a previous kg_get_output_async (its outputs must be complete before the handle's
// buffers are reused). Caller holds h->mu.
int settle(kg_handle* h) {
  if (h->helper.joinable()) h->helper.join();
  return h->helper_status;
}

// copy_inputs (backend.rs:497-546): rows to the pinned staging buffers, with each row's symmetry.
void copy_inputs(kg_handle* h, int n, const kg_row_input* rows) {
  for (int r = 0; r < n; r++) {
    const kg_row_input& in = rows[r];
    if (in.symmetry < 0 || in.symmetry > 7) throw std::runtime_error("kgx backend: symmetry must be in [0, 8)");
    if (!in.row_spatial || (h->nglob && !in.row_global)) throw std::runtime_error("kgx backend: null input row");
    std::memcpy(h->h_glob + (size_t)r * h->nglob, in.row_global, (size_t)h->nglob * 4);
    if (h->nmeta) {
      if (!in.row_meta) throw std::runtime_error("kgx backend: the network needs a meta row");
      std::memcpy(h->h_meta + (size_t)r * h->nmeta, in.row_meta, (size_t)h->nmeta * 4);
    } else if (in.row_meta) {
      throw std::runtime_error("kgx backend: the network takes no meta row");
    }
    copy_with_symmetry(in.row_spatial, h->h_bin + (size_t)r * h->nin * HW, h->nin, POS, POS, in.symmetry, false);
  }
}

// The device post-processing's buffers (first use on the handle). Caller holds h->mu, the handle's device current.
void ensure_post(kg_handle* h) {
  if (h->d_post_out) return;
  const size_t B = (size_t)h->max_batch, rl = (size_t)h->net->row_len();
  KGX_HIP(hipMalloc((void**)&h->d_post_raw, B * rl * 4));
  KGX_HIP(hipMalloc((void**)&h->d_post_rows, B * sizeof(kgx::PostRow)));
  KGX_HIP(hipMalloc((void**)&h->d_legal, B * (HW + 1)));
  KGX_HIP(hipMalloc((void**)&h->d_post_status, B * sizeof(int)));
  KGX_HIP(hipHostMalloc((void**)&h->h_post_rows, B * sizeof(kgx::PostRow), hipHostMallocDefault));
  KGX_HIP(hipHostMalloc((void**)&h->h_legal, B * (HW + 1), hipHostMallocDefault));
  KGX_HIP(hipHostMalloc((void**)&h->h_post_out, B * kgx::POST_LEN * 4, hipHostMallocDefault));
  KGX_HIP(hipHostMalloc((void**)&h->h_post_status, B * sizeof(int), hipHostMallocDefault));
  KGX_HIP(hipMalloc((void**)&h->d_post_out, B * kgx::POST_LEN * 4));
}

// NNEvaluator's inputs of the post-processing per row (nneval.rs:1197-1500), checked, into the pinned staging and
// enqueued to the device.
void stage_post(kg_handle* h, int n, const int* sym, const float* opt, const kg_post_input* post) {
  for (int r = 0; r < n; r++) {
    const kg_post_input& q = post[r];
    if (sym[r] < 0 || sym[r] > 7) throw std::runtime_error("kgx backend: symmetry must be in [0, 8)");
    if (!q.legal) throw std::runtime_error("kgx backend: null legality row");
    if (q.board_x_size < 1 || q.board_x_size > POS || q.board_y_size < 1 || q.board_y_size > POS)
      throw std::runtime_error("kgx backend: board size must be within the 19x19 input");
    if (!(q.nn_policy_temperature > 0.f) || !std::isfinite(q.nn_policy_temperature))
      throw std::runtime_error("kgx backend: nnPolicyTemperature must be positive");
    int legal = 0;
    for (int i = 0; i <= HW; i++) {
      const unsigned char b = q.legal[i] != 0;
      h->h_legal[(size_t)r * (HW + 1) + i] = b;
      legal += b;
    }
    if (legal == 0) throw std::runtime_error("kgx backend: no legal move");  // the reference asserts legal_count > 0
    kgx::PostRow& pr = h->h_post_rows[r];
    pr.symmetry = sym[r];
    pr.optimism = opt[r];
    pr.white_to_move = q.white_to_move != 0;
    pr.board_x = q.board_x_size;
    pr.board_y = q.board_y_size;
    pr.policy_scale = 1.0f / q.nn_policy_temperature;  // outputScaleMultiplier (1) / nnPolicyTemperature, in float
    pr.passing_hacks = q.enable_passing_hacks != 0;
    pr.no_result = q.no_result_allowed != 0;
  }
  KGX_HIP(hipMemcpyAsync(h->d_post_rows, h->h_post_rows, (size_t)n * sizeof(kgx::PostRow), hipMemcpyHostToDevice,
                         h->stream));
  KGX_HIP(hipMemcpyAsync(h->d_legal, h->h_legal, (size_t)n * (HW + 1), hipMemcpyHostToDevice, h->stream));
}

// The post-processing kernel on n raw rows on the device, one readback of its rows and statuses, and the fields
// into the caller's outputs; a nonfinite row fails with the reference's message.
void post_and_read(kg_handle* h, int n, const float* d_raw, kg_nn_output* outputs) {
  kgx::launch_post(d_raw, h->net->row_len(), h->d_post_rows, h->d_legal, h->post_model, h->d_post_out,
                   h->d_post_status, n, h->stream);
  KGX_HIP(hipMemcpyAsync(h->h_post_out, h->d_post_out, (size_t)n * kgx::POST_LEN * 4, hipMemcpyDeviceToHost,
                         h->stream));
  KGX_HIP(hipMemcpyAsync(h->h_post_status, h->d_post_status, (size_t)n * sizeof(int), hipMemcpyDeviceToHost,
                         h->stream));
  KGX_HIP(hipStreamSynchronize(h->stream));
  for (int r = 0; r < n; r++) {
    const int st = h->h_post_status[r];
    if (st & 1) throw std::runtime_error("Got nonfinite for policy sum");
    if (st & 2) throw std::runtime_error("Got nonfinite for nneval value");
  }
  for (int r = 0; r < n; r++) {
    const float* p = h->h_post_out + (size_t)r * kgx::POST_LEN;
    kg_nn_output& o = outputs[r];
    std::memcpy(o.policy_probs, p, (HW + 1) * sizeof(float));
    const float* v = p + HW + 1;
    o.white_win_prob = v[0]; o.white_loss_prob = v[1]; o.white_no_result_prob = v[2];
    o.white_score_mean = v[3]; o.white_score_mean_sq = v[4]; o.white_lead = v[5]; o.var_time_left = v[6];
    o.shortterm_winloss_error = v[7]; o.shortterm_score_error = v[8];
    if (o.white_owner_map) std::memcpy(o.white_owner_map, v + 9, HW * sizeof(float));
  }
}

void upload_rows(kg_handle* h, int n) {
  KGX_HIP(hipMemcpyAsync(h->net->d_bin(), h->h_bin, (size_t)n * h->nin * HW * 4, hipMemcpyHostToDevice, h->stream));
  KGX_HIP(hipMemcpyAsync(h->net->d_global(), h->h_glob, (size_t)n * h->nglob * 4, hipMemcpyHostToDevice, h->stream));
  if (h->nmeta)
    KGX_HIP(hipMemcpyAsync(h->net->d_meta(), h->h_meta, (size_t)n * h->nmeta * 4, hipMemcpyHostToDevice, h->stream));
}

// The device featurizer for n positions into the handle's input buffers, enqueued on its stream (kg_featurize).
// Caller holds h->mu; every position and symmetry is checked before anything is enqueued.
void enqueue_featurize(kg_handle* h, int n, const kg_position* rows, const int* symmetry) {
  if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
  if (h->nin != 22 || h->nglob != 19)
    throw std::runtime_error("kgx featurizer: the network does not take the version-7 inputs (22 spatial and 19 "
                             "global features)");
  for (int r = 0; r < n; r++) {
    kgx::validate_position(rows[r], POS, POS);
    if (symmetry && (symmetry[r] < 0 || symmetry[r] > 7))
      throw std::runtime_error("kgx backend: symmetry must be in [0, 8)");
  }
  KGX_HIP(hipSetDevice(h->device));
  const size_t B = (size_t)h->max_batch;
  if (!h->h_feat) {
    h->feat_sym_bytes = (B * sizeof(int) + 255) / 256 * 256;
    KGX_HIP(hipHostMalloc((void**)&h->h_feat, h->feat_sym_bytes + B * sizeof(kg_position), hipHostMallocDefault));
    KGX_HIP(hipEventCreateWithFlags(&h->pos_uploaded, hipEventDisableTiming));
  }
  // The previous call's kernel must have read the staging before it is overwritten.
  if (h->pos_pending) KGX_HIP(hipEventSynchronize(h->pos_uploaded));
  int* h_sym = (int*)h->h_feat;
  for (int r = 0; r < n; r++) h_sym[r] = symmetry ? symmetry[r] : 0;
  std::memcpy(h->h_feat + h->feat_sym_bytes, rows, (size_t)n * sizeof(kg_position));
  kgx::launch_featurize((const kg_position*)(h->h_feat + h->feat_sym_bytes), n, POS, POS, false, (const int*)h->h_feat,
                        h->net->d_bin(), h->net->d_global(), h->nglob, h->stream);
  KGX_HIP(hipEventRecord(h->pos_uploaded, h->stream));
  h->pos_pending = true;
}

}  // namespace

extern "C" {

const char* kg_version(void) { return "kgx 0.1.0 (gfx950)"; }

const char* kg_last_error(void) { return g_last_error.c_str(); }

int kg_device_count(int* count) {
  return guarded([&] {
    int c = 0;
    KGX_HIP(hipGetDeviceCount(&c));
    *count = c;
  });
}

int kg_device_open(int device) {
  return guarded([&] {
    KGX_HIP(hipSetDevice(device));
    KGX_HIP(hipFree(nullptr));
  });
}

int kg_net_load(const void* model_bytes, size_t len, const char* expected_sha256, kg_net** out) {
  return guarded([&] {
    *out = nullptr;
    if (expected_sha256 && expected_sha256[0])
      throw std::runtime_error("Error loading or parsing model file: expectedSha256 is not supported by the kgx backend");
    if (!model_bytes || len == 0) throw std::runtime_error("Error loading or parsing model file: empty model");
    auto net = std::make_unique<kg_net>();
    net->model = std::make_shared<const kgx::ModelDesc>(kgx::parse_model((const uint8_t*)model_bytes, len));
    *out = net.release();
  });
}

void kg_net_free(kg_net* net) { delete net; }

int kg_net_desc(const kg_net* net, kg_model_desc* d) {
  return guarded([&] {
    if (!net || !d) throw std::runtime_error("null argument");
    const kgx::ModelDesc& m = *net->model;
    std::memset(d, 0, sizeof(*d));
    std::strncpy(d->name, m.name.c_str(), sizeof(d->name) - 1);
    d->model_version = m.version;
    d->num_input_channels = m.num_input_channels;
    d->num_input_global_channels = m.num_global;
    d->num_input_meta_channels = m.num_meta;
    d->num_policy_channels = m.P;
    d->num_value_channels = 3;
    d->num_score_value_channels = m.S;
    d->num_ownership_channels = 1;
    d->trunk_num_channels = m.trunk_c;
    d->trunk_num_blocks = m.trunk_blocks;
    d->num_parameters = m.num_parameters();
    for (int k = 0; k < 7; k++) d->post_process_params[k] = m.post_process[k];
    d->output_row_len = m.row_len();
  });
}

int kg_handle_create(const kg_net* net, int device, int max_batch, int precision, int nn_x_len, int nn_y_len,
                     int inputs_use_nhwc, kg_handle** out) {
  return guarded([&] {
    *out = nullptr;
    if (!net) throw std::runtime_error("null net");
    if (nn_x_len != POS || nn_y_len != POS)
      throw std::runtime_error("kgx backend: nnXLen and nnYLen must equal the network's posLen 19");
    if (inputs_use_nhwc) throw std::runtime_error("kgx backend: inputsUseNHWC = true unsupported");
    if (max_batch < 1) throw std::runtime_error("kgx backend: max batch size must be positive");
    if (precision < KG_PRECISION_F32 || precision > KG_PRECISION_BF16) throw std::runtime_error("kgx backend: unknown precision");
    auto h = std::make_unique<kg_handle>();
    h->device = device;
    h->max_batch = max_batch;
    h->precision = precision;
    const kgx::ModelDesc& m = *net->model;
    // The input buffers' layout must be the model version's (BurnInputBuffers::new, backend.rs:184-188).
    int iv = 0, nsp = 0, ngl = 0;
    model_version_features(m.version, iv, nsp, ngl);
    if (m.num_input_channels != nsp || m.num_global != ngl)
      throw std::runtime_error("kgx backend: model version " + std::to_string(m.version) + " takes " +
                               std::to_string(nsp) + " spatial and " + std::to_string(ngl) +
                               " global input features, the model has " + std::to_string(m.num_input_channels) +
                               " and " + std::to_string(m.num_global));
    if (m.num_meta != meta_encoder_channels(m.meta_version))
      throw std::runtime_error("kgx backend: SGF metadata input must have 192 channels");
    h->model_version = m.version;
    h->P = m.P;
    h->S = m.S;
    h->nin = m.num_input_channels;
    h->nglob = m.num_global;
    h->nmeta = m.num_meta;
    KGX_HIP(hipSetDevice(device));
    KGX_HIP(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
    h->net = std::make_unique<kgx::Net>(m, device, max_batch, precision);
    h->model = net->model;
    KGX_HIP(hipHostMalloc((void**)&h->h_bin, (size_t)max_batch * h->nin * HW * 4, hipHostMallocDefault));
    KGX_HIP(hipHostMalloc((void**)&h->h_glob, (size_t)max_batch * h->nglob * 4, hipHostMallocDefault));
    if (h->nmeta) KGX_HIP(hipHostMalloc((void**)&h->h_meta, (size_t)max_batch * h->nmeta * 4, hipHostMallocDefault));
    // Coherent: the readback kernel's stores go straight to host memory.
    KGX_HIP(hipHostMalloc((void**)&h->h_out, (size_t)max_batch * m.row_len() * 4, hipHostMallocCoherent));
    h->post_model.P = h->P;
    h->post_model.S = h->S;
    h->post_model.version = h->model_version;
    // ModelPostProcessParams: the model file's floats widened to double (bin2onnx.py:1025-1031).
    for (int k = 0; k < 7; k++) h->post_model.pp[k] = (double)m.post_process[k];
    std::memset(h->h_bin, 0, (size_t)max_batch * h->nin * HW * 4);
    std::memset(h->h_glob, 0, (size_t)max_batch * h->nglob * 4);
    if (h->nmeta) std::memset(h->h_meta, 0, (size_t)max_batch * h->nmeta * 4);
    *out = h.release();
  });
}

void kg_handle_free(kg_handle* h) {
  if (!h) return;
  {
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
  }
  (void)hipSetDevice(h->device);
  if (h->stream) (void)hipStreamSynchronize(h->stream);
  h->net.reset();
  if (h->h_bin) (void)hipHostFree(h->h_bin);
  if (h->h_glob) (void)hipHostFree(h->h_glob);
  if (h->h_meta) (void)hipHostFree(h->h_meta);
  if (h->h_out) (void)hipHostFree(h->h_out);
  if (h->d_post_raw) (void)hipFree(h->d_post_raw);
  if (h->d_post_rows) (void)hipFree(h->d_post_rows);
  if (h->d_legal) (void)hipFree(h->d_legal);
  if (h->d_post_out) (void)hipFree(h->d_post_out);
  if (h->d_post_status) (void)hipFree(h->d_post_status);
  if (h->h_post_rows) (void)hipHostFree(h->h_post_rows);
  if (h->h_legal) (void)hipHostFree(h->h_legal);
  if (h->h_post_out) (void)hipHostFree(h->h_post_out);
  if (h->h_post_status) (void)hipHostFree(h->h_post_status);
  if (h->h_feat) (void)hipHostFree(h->h_feat);
  if (h->pos_uploaded) (void)hipEventDestroy(h->pos_uploaded);
  if (h->stream) (void)hipStreamDestroy(h->stream);
  delete h;
}

int kg_handle_set_batch_buckets(kg_handle* h, const int* buckets, int count) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (count > 0 && !buckets) throw std::runtime_error("null buckets");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    h->buckets.clear();
    for (int k = 0; k < count; k++)
      if (buckets[k] > 0) h->buckets.push_back(buckets[k]);
    std::sort(h->buckets.begin(), h->buckets.end());
    h->buckets.erase(std::unique(h->buckets.begin(), h->buckets.end()), h->buckets.end());
  });
}

int kg_padded_batch_size(const int* buckets, int count, int n, int max_batch) {
  std::vector<int> b(buckets, buckets + (count > 0 ? count : 0));
  return padded_batch_size(b, n, max_batch);
}

int kg_copy_with_symmetry(const float* src, float* dst, int channels, int h, int w, int symmetry, int reverse) {
  return guarded([&] {
    if (!src || !dst) throw std::runtime_error("null buffer");
    if (channels < 1 || h < 1 || w < 1) throw std::runtime_error("bad plane shape");
    if (symmetry < 0 || symmetry > 7) throw std::runtime_error("symmetry must be in [0, 8)");
    copy_with_symmetry(src, dst, channels, h, w, symmetry, reverse != 0);
  });
}

int kg_conv_geometry(int ks, int ic, int oc, int split, int pixels, kg_conv_geometry_t* out) {
  return guarded([&] {
    if (!out) throw std::runtime_error("null output");
    if ((ks != 1 && ks != 3) || ic < 1 || oc < 1 || pixels < 1 || (split && ks != 1))
      throw std::runtime_error("bad convolution shape");
    const kgx::IgemmGeometry g = kgx::conv_igemm_geometry(ks, ic, oc, split != 0, pixels);
    *out = kg_conv_geometry_t{g.grid, g.threads, g.tile_rows, g.tile_cols, g.stage_channels, g.pixel_tiles,
                              g.col_tiles, g.pairs, g.weights_direct, g.weight_rows, g.waves,
                              g.direct_instructions, g.direct_per_wave};
  });
}

int kg_conv_tile_of(int ks, int ic, int oc, int split, int pixels, int workgroup, int* pixel_tile, int* col_tile) {
  return guarded([&] {
    if (!pixel_tile || !col_tile) throw std::runtime_error("null output");
    if ((ks != 1 && ks != 3) || ic < 1 || oc < 1 || pixels < 1 || (split && ks != 1))
      throw std::runtime_error("bad convolution shape");
    const kgx::IgemmGeometry g = kgx::conv_igemm_geometry(ks, ic, oc, split != 0, pixels);
    if (workgroup < 0 || workgroup >= g.grid) throw std::runtime_error("workgroup out of range");
    kgx::conv_igemm_tile_of(g, workgroup, *pixel_tile, *col_tile);
  });
}

int kg_junction_tile_of(int pixels, int workgroup, int* grid, int* tile) {
  return guarded([&] {
    if (!grid || !tile) throw std::runtime_error("null output");
    if (pixels < 1) throw std::runtime_error("bad pixel count");
    *grid = kgx::junction_grid(pixels);
    if (workgroup < 0 || workgroup >= *grid) throw std::runtime_error("workgroup out of range");
    const int t = kgx::junction_tile_of(workgroup);
    *tile = t * 48 < pixels ? t : -1;
  });
}

int kg_gpool_tile_of(int pixels, int gpool_channels, int regular_channels, int workgroup, int* grid, int* tile,
                     int* first_channel, int* channels) {
  return guarded([&] {
    if (!grid || !tile || !first_channel || !channels) throw std::runtime_error("null output");
    if (pixels < 1) throw std::runtime_error("bad pixel count");
    const int share = kgx::gpool_tile_share(gpool_channels, regular_channels);
    if (!share) throw std::runtime_error("no tile share fits these channel counts");
    const int shares = regular_channels / share;
    *grid = kgx::gpool_tile_grid(pixels, shares);
    if (workgroup < 0 || workgroup >= *grid) throw std::runtime_error("workgroup out of range");
    int t, s;
    kgx::gpool_tile_of(workgroup, shares, t, s);
    *tile = t * kgx::kGpoolTileRows < pixels ? t : -1;
    *first_channel = s * share;
    *channels = share;
  });
}

int kg_l2_touch_line(int grid, int workgroup, int thread, int* line) {
  return guarded([&] {
    if (!line) throw std::runtime_error("null output");
    if (grid < 1 || workgroup < 0 || workgroup >= grid || thread < 0) throw std::runtime_error("bad launch index");
    *line = kgx::l2_touch_line(workgroup, grid, thread);
  });
}

int kg_rmsnorm_rows_of(int rows, int channels, int region, int workgroup, int* grid, int* first_row, int* count) {
  return guarded([&] {
    if (!grid || !first_row || !count) throw std::runtime_error("null output");
    if (rows < 1 || region < 0) throw std::runtime_error("bad row count or tile");
    const int per_wg = kgx::rmsnorm_rows_per_workgroup(channels);
    if (!per_wg) throw std::runtime_error("this channel count takes the scalar RMSNorm kernel");
    if (region % per_wg) region = 0;
    *grid = kgx::rmsnorm_grid(rows, region, per_wg);
    if (workgroup < 0 || workgroup >= *grid) throw std::runtime_error("workgroup out of range");
    const int f = kgx::rmsnorm_first_row(workgroup, region, per_wg);
    *first_row = f;
    *count = f < rows ? std::min(per_wg, rows - f) : 0;
  });
}

int kg_conv_weight_load(int ks, int ic, int oc, int split, int q, int wave, int lane, int* src_row, int* src_chunk,
                        int* dst_row, int* dst_chunk) {
  return guarded([&] {
    if (!src_row || !src_chunk || !dst_row || !dst_chunk) throw std::runtime_error("null output");
    if ((ks != 1 && ks != 3) || ic < 1 || oc < 1 || (split && ks != 1)) throw std::runtime_error("bad convolution shape");
    const kgx::IgemmGeometry g = kgx::conv_igemm_geometry(ks, ic, oc, split != 0, 1);
    if (!g.weights_direct) throw std::runtime_error("this convolution stages its weights through registers");
    if (q < 0 || q >= g.direct_per_wave || wave < 0 || wave >= g.waves || lane < 0 || lane >= 64)
      throw std::runtime_error("direct load index out of range");
    kgx::conv_igemm_weight_load(g, q, wave, lane, *src_row, *src_chunk, *dst_row, *dst_chunk);
  });
}

int kg_conv_weight_chunk(int row, int chunk) {
  return row >= 0 && chunk >= 0 && chunk < 8 ? kgx::conv_igemm_weight_chunk(row, chunk) : -1;
}

int kg_handle_is_using_fp16(const kg_handle* h) { return h && h->precision != KG_PRECISION_F32 ? 1 : 0; }

int kg_forward(kg_handle* h, int n, const float* bin, const float* global, const float* meta, float* out) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!bin || (h->nglob && !global) || !out) throw std::runtime_error("kgx backend: null input or output buffer");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
    if (h->nmeta && !meta) throw std::runtime_error("kgx backend: the network needs a meta_input");
    if (!h->nmeta && meta) throw std::runtime_error("kgx backend: the network takes no meta_input");
    const int n_run = padded_batch_size(h->buckets, n, h->max_batch);
    std::memcpy(h->h_bin, bin, (size_t)n * h->nin * HW * 4);
    std::memcpy(h->h_glob, global, (size_t)n * h->nglob * 4);
    if (h->nmeta) std::memcpy(h->h_meta, meta, (size_t)n * h->nmeta * 4);
    KGX_HIP(hipSetDevice(h->device));
    upload_rows(h, n);
    run_and_read(h, n_run, n, out);
  });
}

int kg_handle_device_buffers(kg_handle* h, float** bin, float** global, float** meta, float** out) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (bin) *bin = h->net->d_bin();
    if (global) *global = h->net->d_global();
    if (meta) *meta = h->net->d_meta();
    if (out) *out = h->net->d_out();
  });
}

int kg_run(kg_handle* h, int n, float* out) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
    KGX_HIP(hipSetDevice(h->device));
    const int n_run = padded_batch_size(h->buckets, n, h->max_batch);
    if (out) run_and_read(h, n_run, n, out);
    else h->net->forward(n_run, h->stream);
  });
}

int kg_run_static(kg_handle* h, int n) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    const int mib = (int)(kgx::kStaticScratchBytes >> 20);
    KGX_HIP(hipSetDevice(h->device));
    if (h->static_batch < 0) plan_static(h, *h->model);
    if (!h->net_static)
      throw std::runtime_error("kgx backend: one row of this network needs more workspace than the static scratch (" +
                               std::to_string(mib) + " MiB)");
    if (n < 1 || n > h->static_batch)
      throw std::runtime_error("kgx backend: batch size " + std::to_string(n) + " out of range for the static scratch (" +
                               std::to_string(mib) + " MiB holds the workspace of at most " +
                               std::to_string(h->static_batch) + " rows of this network)");
    h->net_static->forward_eager(padded_batch_size(h->buckets, n, h->static_batch), h->stream);
  });
}

int kg_sync(kg_handle* h) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    {
      std::lock_guard<std::mutex> lock(h->mu);
      settle(h);
    }
    KGX_HIP(hipStreamSynchronize(h->stream));
  });
}

void* kg_handle_stream(kg_handle* h) { return h ? (void*)h->stream : nullptr; }

int kg_get_output(kg_handle* h, int n, const kg_row_input* rows, kg_nn_output* outputs) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!rows || !outputs) throw std::runtime_error("null rows or outputs");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
    copy_inputs(h, n, rows);
    // run_network (backend.rs:549-619).
    KGX_HIP(hipSetDevice(h->device));
    const int n_run = padded_batch_size(h->buckets, n, h->max_batch);
    upload_rows(h, n);
    run_and_read(h, n_run, n, nullptr);
    // copy_outputs (backend.rs:622-731).
    const int rl = h->net->row_len();
    for (int r = 0; r < n; r++)
      copy_outputs_row(h->h_out + (size_t)r * rl, h->P, h->S, h->model_version, rows[r].symmetry,
                       rows[r].policy_optimism, outputs[r]);
  });
}

int kg_get_output_eval(kg_handle* h, int n, const kg_row_input* rows, const kg_post_input* post,
                       kg_nn_output* outputs) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!rows || !post || !outputs) throw std::runtime_error("null rows, post-processing inputs or outputs");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
    copy_inputs(h, n, rows);
    std::vector<int> sym(n);
    std::vector<float> opt(n);
    for (int r = 0; r < n; r++) {
      sym[r] = rows[r].symmetry;
      opt[r] = rows[r].policy_optimism;
    }
    KGX_HIP(hipSetDevice(h->device));
    ensure_post(h);
    stage_post(h, n, sym.data(), opt.data(), post);
    const int n_run = padded_batch_size(h->buckets, n, h->max_batch);
    upload_rows(h, n);
    h->net->forward(n_run, h->stream);
    post_and_read(h, n, h->net->d_out(), outputs);
  });
}

int kg_featurize(kg_handle* h, int n, const kg_position* rows, const int* symmetry) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!rows) throw std::runtime_error("null positions");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    enqueue_featurize(h, n, rows, symmetry);
  });
}

int kg_evaluate_positions(kg_handle* h, int n, const kg_position* rows, const int* symmetry,
                          const float* policy_optimism, const kg_post_input* post, kg_nn_output* outputs) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!rows || !post || !outputs) throw std::runtime_error("null positions, post-processing inputs or outputs");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (h->nmeta) throw std::runtime_error("kgx featurizer: the network takes metadata inputs, which it does not write");
    enqueue_featurize(h, n, rows, symmetry);
    std::vector<int> sym(n, 0);
    std::vector<float> opt(n, 0.f);
    for (int r = 0; r < n; r++) {
      if (symmetry) sym[r] = symmetry[r];
      if (policy_optimism) opt[r] = policy_optimism[r];
    }
    ensure_post(h);
    stage_post(h, n, sym.data(), opt.data(), post);
    h->net->forward(padded_batch_size(h->buckets, n, h->max_batch), h->stream);
    post_and_read(h, n, h->net->d_out(), outputs);
  });
}

int kg_featurize_rows(int device, int n, const kg_position* rows, int nn_x_len, int nn_y_len, int use_nhwc,
                      const int* symmetry, float* bin, float* global) {
  return guarded([&] {
    if (!rows || !bin || !global) throw std::runtime_error("null argument");
    if (n < 1) throw std::runtime_error("kgx featurizer: no positions");
    if (nn_x_len < 1 || nn_y_len < 1 || nn_x_len > POS || nn_y_len > POS)
      throw std::runtime_error("kgx featurizer: nn_x_len and nn_y_len must be in [1, 19]");
    for (int r = 0; r < n; r++) {
      kgx::validate_position(rows[r], nn_x_len, nn_y_len);
      if (symmetry && (symmetry[r] < 0 || symmetry[r] > 7))
        throw std::runtime_error("kgx backend: symmetry must be in [0, 8)");
    }
    KGX_HIP(hipSetDevice(device));
    const size_t row = (size_t)22 * nn_x_len * nn_y_len;
    kgx::DeviceBuffer d_pos, d_sym, d_bin, d_glob;  // freed on every exit
    KGX_HIP(hipMalloc(&d_pos.ptr, (size_t)n * sizeof(kg_position)));
    KGX_HIP(hipMalloc(&d_sym.ptr, (size_t)n * sizeof(int)));
    KGX_HIP(hipMalloc(&d_bin.ptr, (size_t)n * row * 4));
    KGX_HIP(hipMalloc(&d_glob.ptr, (size_t)n * 19 * 4));
    std::vector<int> sym(n, 0);
    if (symmetry) std::copy(symmetry, symmetry + n, sym.begin());
    KGX_HIP(hipMemcpy(d_pos.ptr, rows, (size_t)n * sizeof(kg_position), hipMemcpyHostToDevice));
    KGX_HIP(hipMemcpy(d_sym.ptr, sym.data(), (size_t)n * sizeof(int), hipMemcpyHostToDevice));
    kgx::launch_featurize((const kg_position*)d_pos.ptr, n, nn_x_len, nn_y_len, use_nhwc != 0, (const int*)d_sym.ptr,
                          (float*)d_bin.ptr, (float*)d_glob.ptr, 19, nullptr);
    KGX_HIP(hipMemcpy(bin, d_bin.ptr, (size_t)n * row * 4, hipMemcpyDeviceToHost));
    KGX_HIP(hipMemcpy(global, d_glob.ptr, (size_t)n * 19 * 4, hipMemcpyDeviceToHost));
  });
}

int kg_post_outputs(kg_handle* h, int n, const float* raw, const int* symmetry, const float* policy_optimism,
                    const kg_post_input* post, kg_nn_output* outputs) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!raw || !symmetry || !policy_optimism || !post || !outputs) throw std::runtime_error("null argument");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
    KGX_HIP(hipSetDevice(h->device));
    ensure_post(h);
    stage_post(h, n, symmetry, policy_optimism, post);
    const size_t bytes = (size_t)n * h->net->row_len() * 4;
    std::memcpy(h->h_out, raw, bytes);
    KGX_HIP(hipMemcpyAsync(h->d_post_raw, h->h_out, bytes, hipMemcpyHostToDevice, h->stream));
    post_and_read(h, n, h->d_post_raw, outputs);
  });
}

int kg_get_output_async(kg_handle* h, int n, const kg_row_input* rows, kg_nn_output* outputs, kg_done_fn done,
                        void* user) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    if (!rows || !outputs) throw std::runtime_error("null rows or outputs");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    if (n < 1 || n > h->max_batch) throw std::runtime_error("kgx backend: batch size out of range");
    // copy_inputs on the calling thread (the inputs are read before the call returns), then the whole batch is
    // enqueued: uploads, the forward pass, one readback into the pinned output rows.
    copy_inputs(h, n, rows);
    std::vector<int> sym(n);
    std::vector<float> opt(n);
    for (int r = 0; r < n; r++) {
      sym[r] = rows[r].symmetry;
      opt[r] = rows[r].policy_optimism;
    }
    KGX_HIP(hipSetDevice(h->device));
    const int n_run = padded_batch_size(h->buckets, n, h->max_batch);
    upload_rows(h, n);
    h->net->forward(n_run, h->stream);
    kgx::launch_readback(h->net->d_out(), h->h_out, (size_t)n * h->net->row_len(), h->stream);
    // read_on_helper_thread (backend.rs:743-753): a fresh OS thread waits for the device and runs copy_outputs.
    h->helper_status = 0;
    h->helper_error.clear();
    h->helper = std::thread([h, n, outputs, done, user, sym = std::move(sym), opt = std::move(opt)] {
      int st = 0;
      try {
        KGX_HIP(hipSetDevice(h->device));
        KGX_HIP(hipStreamSynchronize(h->stream));
        const int rl = h->net->row_len();
        for (int r = 0; r < n; r++)
          copy_outputs_row(h->h_out + (size_t)r * rl, h->P, h->S, h->model_version, sym[r], opt[r], outputs[r]);
      } catch (const std::exception& e) {
        st = 1;
        h->helper_error = std::string("kgx backend: readback failed: ") + e.what();
      }
      h->helper_status = st;
      if (done) done(user, st);
    });
  });
}

int kg_wait(kg_handle* h) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    if (settle(h) != 0) {
      const std::string msg = h->helper_error;
      h->helper_status = 0;
      throw std::runtime_error(msg);
    }
  });
}

int kg_copy_outputs(const float* raw, int n, int P, int S, int model_version, const int* symmetry,
                    const float* policy_optimism, kg_nn_output* outputs) {
  return guarded([&] {
    if (!raw || !symmetry || !policy_optimism || !outputs) throw std::runtime_error("null argument");
    if (n < 0) throw std::runtime_error("negative row count");
    int iv, sp, gl;
    model_version_features(model_version, iv, sp, gl);
    if (!(P == 1 || P == 2 || P == 4)) throw std::runtime_error("policy channels must be 1, 2 or 4");
    if (S != score_channels_for_version(model_version))
      throw std::runtime_error("score value channels do not match the model version");
    const size_t rl = (size_t)P * (HW + 1) + 3 + S + HW;
    for (int r = 0; r < n; r++) {
      if (symmetry[r] < 0 || symmetry[r] > 7) throw std::runtime_error("symmetry must be in [0, 8)");
      copy_outputs_row(raw + r * rl, P, S, model_version, symmetry[r], policy_optimism[r], outputs[r]);
    }
  });
}

int kg_model_version_features(int model_version, int* inputs_version, int* num_spatial, int* num_global) {
  return guarded([&] {
    int iv, sp, gl;
    model_version_features(model_version, iv, sp, gl);
    if (inputs_version) *inputs_version = iv;
    if (num_spatial) *num_spatial = sp;
    if (num_global) *num_global = gl;
  });
}

int kg_meta_encoder_channels(int meta_encoder_version, int* num_meta) {
  return guarded([&] {
    const int c = meta_encoder_channels(meta_encoder_version);
    if (num_meta) *num_meta = c;
  });
}

int kg_profile_enable(kg_handle* h, int enable) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    h->net->set_profiling(enable != 0);
  });
}

int kg_profile_reset(kg_handle* h) {
  return guarded([&] {
    if (!h) throw std::runtime_error("null handle");
    std::lock_guard<std::mutex> lock(h->mu);
    settle(h);
    h->net->reset_profile();
  });
}

int kg_profile_read(kg_handle* h, const char** names, long* launches, double* ms, double* flops, double* bytes,
                    int max_classes) {
  if (!h) return -1;
  std::lock_guard<std::mutex> lock(h->mu);
  int k = 0;
  for (const auto& kv : h->net->profile()) {
    if (k < max_classes) {
      names[k] = kv.second.name;
      launches[k] = kv.second.launches;
      ms[k] = kv.second.ms;
      flops[k] = kv.second.flops;
      bytes[k] = kv.second.bytes;
    }
    k++;
  }
  return k;
}

}  // extern "C"
