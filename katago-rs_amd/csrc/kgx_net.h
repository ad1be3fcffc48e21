// A KataGo network on one GPU: device weights in the layouts the kernels read, activation workspace for a
// maximum batch, and the forward pass as a list of kernel launches (replayed through a HIP graph per batch
// size, or launched eagerly with per-kernel events when profiling).
#pragma once
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "kgx_kernels.h"
#include "kgx_model.h"

namespace kgx {

#define KGX_HIP(call)                                                                                       \
  do {                                                                                                      \
    hipError_t e_ = (call);                                                                                 \
    if (e_ != hipSuccess) throw std::runtime_error(std::string(#call) + ": " + hipGetErrorString(e_));    \
  } while (0)

struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
};

// One kernel launch of the forward pass. Work is algorithmic (what the operation must read, write and compute),
// linear in the batch: per_row * B + fixed.
struct Op {
  std::function<void(hipStream_t, int)> launch;
  const char* cls;
  double flops_row = 0, bytes_row = 0, bytes_fixed = 0;
  // A convolution / GEMM output whose emission may be attached after the op is planned: its compute-type
  // activation of `out_c` channels per point is counted when present.
  std::shared_ptr<ConvOut> out;
  int out_c = 0;
  // Weights that every XCD reads (an implicit-GEMM convolution's or a junction's), and the output descriptor through
  // which the op's kernel touches the next such op's weights into L2 (ConvOut::pf).
  const void* w = nullptr; size_t w_bytes = 0;
  std::shared_ptr<ConvOut> pf_sink;
};

// Planning state of one residual stream (the trunk, or the inner stream of a nested bottleneck block): its float
// values, the two compute-type buffers that its consumer activations alternate between (so a producer never
// writes the buffer its own input was read from) with their low planes for split-operand consumers (allocated on
// first use), and the op that last wrote the stream, which emits the next consumer's activation.
struct StreamState {
  float* x = nullptr;
  int c = 0;
  void* act[2] = {nullptr, nullptr};
  void* act_lo[2] = {nullptr, nullptr};
  int flip = 0;
  std::shared_ptr<ConvOut> producer;
};

struct ProfileClass {
  const char* name = nullptr;  // the op table's string literal
  long launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};

class Net {
 public:
  Net(const ModelDesc& model, int device, int max_batch, int prec);
  // A second plan of `primary`'s network that allocates nothing: its weights are the primary's (uploaded in the
  // same order), its inputs and outputs are the primary's device buffers, and its workspace is bump-allocated
  // from [ws_base, ws_base + ws_cap) (the planning only records addresses; fits() tells whether they stayed
  // within the capacity).
  Net(const ModelDesc& model, const Net& primary, int max_batch, char* ws_base, size_t ws_cap);
  ~Net();

  // Enqueues the forward pass over the first B rows of the device input buffers on `stream`.
  void forward(int B, hipStream_t stream);
  // The forward pass of a workspace plan (second constructor): eager launches only (no graph capture, no event,
  // no allocation), after clearing the workspace regions the planning zeroes once in a primary plan.
  void forward_eager(int B, hipStream_t stream);
  bool fits() const { return ws_used_ <= ws_cap_; }
  size_t workspace_bytes() const { return ws_used_; }

  int prec() const { return prec_; }
  int max_batch() const { return max_batch_; }
  int row_len() const { return row_len_; }
  float* d_bin() const { return d_bin_; }
  float* d_global() const { return d_glob_; }
  float* d_meta() const { return d_meta_; }
  float* d_out() const { return d_out_; }
  size_t bin_row() const { return (size_t)nin_ * HW; }
  int num_global() const { return nglob_; }
  int num_meta() const { return nmeta_; }

  void set_profiling(bool on) { profiling_ = on; }
  void reset_profile() { profile_.clear(); }
  const std::map<std::string, ProfileClass>& profile() const { return profile_; }
  void set_use_graphs(bool on) { use_graphs_ = on; }

 private:
  // Allocation and upload. A workspace plan (primary_ set) bump-allocates workspace and takes the primary's
  // uploads in order.
  float* alloc_f(size_t n);
  void* alloc_bytes(size_t bytes);
  const float* upload_f(const std::vector<float>& v);
  // A row-program matrix and its bias as one upload (the bias right after W, padded to 16 bytes), so that the
  // program's weight staging copies the bias with W.
  void upload_mm(RowMM& mm, const std::vector<float>& w, const std::vector<float>& b);
  const void* take_upload(size_t bytes);
  const void* upload_t(const std::vector<float>& v);  // converted to the compute type
  size_t tsize() const { return prec_ == PREC_F32 ? 4 : 2; }

  // Planning.
  void scan(const std::vector<BlockDesc>& blocks, int c, int depth);
  // Whether conv c runs as an implicit GEMM (16-bit handles, 1x1 / 3x3, channel and stride alignment).
  bool igemm_eligible(const ConvDesc& c, bool nchw, int ldx, const ConvOut& o) const;
  // conv(x) into `o`; x is a compute-type activation [rows][ldx], or the float NCHW network input. With x_lo (the
  // low plane of a split activation) the convolution runs on split operands.
  std::shared_ptr<ConvOut> emit_conv(const ConvDesc& c, const void* x, int ldx, bool nchw, const ConvOut& o,
                                     const void* x_lo = nullptr);
  // Whether a 1x1 convolution over a stream activation runs on split operands: on 16-bit handles every
  // implicit-GEMM 1x1 does, so that only 3x3 convolutions round their operands to 16 bits.
  bool split_1x1(const ConvDesc& c, int ldx, const ConvOut& o) const;
  void emit_stack(const std::vector<BlockDesc>& blocks, int depth);
  // A nested block's exit convolution held back while the next block's entry is planned: both then run as one
  // junction launch (launch_junction), which keeps the activation between them in LDS.
  struct PendingExit {
    const ConvDesc* conv = nullptr;
    const void* x = nullptr;
    const void* x_lo = nullptr;
    int ldx = 0;
    std::shared_ptr<ConvOut> out;
    bool stem = false;  // the network's stem (x: the packed input rows), joined with the first block's entry
  };
  // Whether block b's exit (over a trunk of c channels) can start a junction, and whether it and block `next`'s entry
  // run as one.
  bool exit_fits(const BlockDesc& b, int c) const;
  bool junction_fits(const BlockDesc& b, const BlockDesc& next, int c) const;
  // Whether the stem (into stem_out) and the first block's entry run as one stem junction.
  bool stem_junction_fits(const ModelDesc& m, const ConvOut& stem_out) const;
  // The input packing launch of a stem convolution c over the float NCHW input x; icin: the packed channels.
  const void* emit_input_pack(const ConvDesc& c, const void* x, int& icin);
  std::shared_ptr<ConvOut> emit_junction(const PendingExit& p, const ConvDesc& entry, const ConvOut& entry_o);
  void emit_attention(const BlockDesc& b, int depth);
  void emit_ffn(const BlockDesc& b, int depth);
  std::shared_ptr<ConvOut> emit_token_gemm(const void* A, int lda, const void* Bt, int N, int K, const ConvOut& o,
                                           const char* cls, bool glu = false, const QkvEpi& qkv = QkvEpi(),
                                           int yt_act = ACT_ID);
  // The activation act(bn(x)) * mask of stream `depth`, emitted by the stream's last producer; with `lo`, also its
  // low plane (split operands), returned there.
  void* consume(int depth, const BNDesc& bn, int act, const void** lo = nullptr);
  Emit bn_emit(const BNDesc& bn, int act, void* out, int ld);
  Prologue bn_pro(const BNDesc& bn, int act, const float* prebias = nullptr, int ld_prebias = 0);
  RowProg row_prog_base() const;  // a row program with the board statistics filled in
  void build(const ModelDesc& m);

  void run_ops(int B, hipStream_t s);

  int t_pad(int B) const;  // Winograd tiles of B rows, padded to the GEMM's row tile

  enum ConvMode { CONV_IGEMM, CONV_WINO2, CONV_WINO4 };
  int device_, max_batch_, prec_;
  const Net* primary_ = nullptr;
  std::vector<std::pair<const void*, size_t>> uploads_;  // device copies of the weights, in upload order
  size_t upload_next_ = 0;                               // workspace plan: the next primary upload to take
  char* ws_base_ = nullptr;
  size_t ws_cap_ = 0, ws_used_ = 0;
  std::vector<std::pair<void*, size_t>> zero_;           // workspace regions cleared before every eager forward
  ConvMode conv_mode_ = CONV_WINO4;
  bool junctions_ = true;  // nested-bottleneck junctions in one launch (KGX_JUNCTION=0: two launches)
  bool head_junction_ = false;  // the trunk's last exit may join the heads' first convolution
  bool l2_prefetch_ = true;  // kernels touch the next op's weights into L2 (KGX_L2_PREFETCH=0: off)
  bool gpool_tile_ = true;   // gpool blocks' mid activation per pixel tile (KGX_GPOOL_TILE=0: per row)
  std::unique_ptr<PendingExit> pend_;
  // The token GEMM that last added into a residual stream (its N and K; 0 when another op wrote the stream last): the
  // RMSNorm that reads the stream next takes its rows in that GEMM's row tiles, on the XCDs that wrote them.
  int res_n_ = 0, res_k_ = 0;
  int wino_tm_ = 4;
  int nin_ = 0, nglob_ = 0, nmeta_ = 0, row_len_ = 0;
  std::vector<std::unique_ptr<DeviceBuffer>> mem_;
  std::vector<Op> ops_;

  // Inputs / outputs and per-row board data.
  float *d_bin_ = nullptr, *d_glob_ = nullptr, *d_meta_ = nullptr, *d_out_ = nullptr;
  InputGlobal stem_glob_;  // the stem's global-input bias, computed in the input packing launch when set
  float *mask_ = nullptr, *area_ = nullptr, *s1_ = nullptr, *s2_ = nullptr;

  // Workspace sizes from scan(), then the buffers.
  int tmp_c_ = 0, mid_c_ = 0, gb_c_ = 0;
  std::vector<int> stream_c_;
  int nrm_c_ = 0, qkv_c_ = 0, ao_c_ = 0, u_c_ = 0, h_c_ = 0;
  size_t wino_v_elems_ = 0, wino_m_elems_ = 0;
  float* trunk_ = nullptr;
  std::vector<StreamState> ss_;
  void* mid_ = nullptr;  // compute-type mid activation of a residual block
  float *tmp_ = nullptr, *gb_ = nullptr;
  void *nrm_ = nullptr, *qkv_ = nullptr, *ao_ = nullptr, *h_ = nullptr;
  float* u_ = nullptr;
  void* wino_v_ = nullptr;
  float* wino_m_ = nullptr;

  bool profiling_ = false, use_graphs_ = true;
  std::map<std::string, ProfileClass> profile_;
  std::vector<hipEvent_t> events_;
  std::map<int, hipGraphExec_t> graphs_;
};

}  // namespace kgx
