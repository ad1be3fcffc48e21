// Forward-pass planning and execution on one GPU. The op order follows the graph of
// tools/bin2onnx/bin2onnx.py (trunk :1466-1492, blocks :1243-1269 and :1357-1438, heads :1495-1531). Each
// batch norm + activation + mask that feeds a convolution (what katago-nn-burn's `fuse_bn_act` rewrite folds into
// the convolution's input, crates/katago-nn-burn/build.rs:366-600, conv.rs:42-93) is computed once, in the
// epilogue of the op that produced its input, and stored in the compute type: the convolution reads half the
// bytes of the float stream and recomputes nothing.
#include "kgx_net.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>

namespace kgx {

namespace {

uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

uint16_t f32_to_bf16_bits(float f) {  // round to nearest even
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

}  // namespace

Net::Net(const ModelDesc& m, int device, int max_batch, int prec) : device_(device), max_batch_(max_batch), prec_(prec) {
  KGX_HIP(hipSetDevice(device));
  // Convolution algorithm. Float operands: Winograd F(4x4,3x3), the reference's. 16-bit operands: implicit GEMM
  // for 1x1 and 3x3 (no transform traffic; only activations and weights are rounded). KGX_CONV=igemm|wino2|wino4
  // overrides (igemm needs 16-bit operands; wino2 is F(2x2,3x3), whose transformed values stay small enough for
  // 16-bit operands).
  conv_mode_ = prec == PREC_F32 ? CONV_WINO4 : CONV_IGEMM;
  if (const char* e = std::getenv("KGX_CONV")) {
    const std::string v = e;
    if (v == "wino4") conv_mode_ = CONV_WINO4;
    else if (v == "wino2") conv_mode_ = CONV_WINO2;
    else if (v == "igemm" && prec != PREC_F32) conv_mode_ = CONV_IGEMM;
  }
  wino_tm_ = conv_mode_ == CONV_WINO4 ? 4 : 2;
  // Nested-bottleneck junctions in one launch; KGX_JUNCTION=0 plans the two convolutions separately.
  if (const char* e = std::getenv("KGX_JUNCTION")) junctions_ = std::string(e) != "0";
  // Each convolution touches the next one's weights into L2 during its epilogue; KGX_L2_PREFETCH=0 turns it off.
  if (const char* e = std::getenv("KGX_L2_PREFETCH")) l2_prefetch_ = std::string(e) != "0";
  // A global-pooling block's mid activation per pixel tile; KGX_GPOOL_TILE=0 plans the per-row program instead.
  if (const char* e = std::getenv("KGX_GPOOL_TILE")) gpool_tile_ = std::string(e) != "0";
  build(m);
}

Net::Net(const ModelDesc& m, const Net& primary, int max_batch, char* ws_base, size_t ws_cap)
    : device_(primary.device_), max_batch_(max_batch), prec_(primary.prec_), primary_(&primary), ws_base_(ws_base),
      ws_cap_(ws_cap) {
  if (max_batch < 1 || max_batch > primary.max_batch_) throw std::runtime_error("internal: workspace plan batch");
  conv_mode_ = primary.conv_mode_;
  wino_tm_ = primary.wino_tm_;
  junctions_ = primary.junctions_;
  l2_prefetch_ = primary.l2_prefetch_;
  gpool_tile_ = primary.gpool_tile_;
  build(m);
  if (upload_next_ != primary.uploads_.size()) throw std::runtime_error("internal: workspace plan weights differ");
}

int Net::t_pad(int B) const { return round_up(B * wino_tiles(wino_tm_), 128); }

Net::~Net() {
  (void)hipSetDevice(device_);
  for (auto& kv : graphs_) (void)hipGraphExecDestroy(kv.second);
  for (hipEvent_t e : events_) (void)hipEventDestroy(e);
}

float* Net::alloc_f(size_t n) { return (float*)alloc_bytes(n * sizeof(float)); }

void* Net::alloc_bytes(size_t bytes) {
  bytes = std::max<size_t>(bytes, 256);
  if (primary_) {
    // Workspace plan: addresses only, 256-byte aligned; the caller checks fits() before running it.
    const size_t off = (ws_used_ + 255) / 256 * 256;
    ws_used_ = off + bytes;
    return ws_base_ + off;
  }
  auto b = std::make_unique<DeviceBuffer>();
  KGX_HIP(hipMalloc(&b->ptr, bytes));
  b->bytes = bytes;
  void* p = b->ptr;
  mem_.push_back(std::move(b));
  return p;
}

const void* Net::take_upload(size_t bytes) {
  if (upload_next_ >= primary_->uploads_.size() || primary_->uploads_[upload_next_].second != bytes)
    throw std::runtime_error("internal: workspace plan weights differ");
  return primary_->uploads_[upload_next_++].first;
}

const float* Net::upload_f(const std::vector<float>& v) {
  if (primary_) return (const float*)take_upload(v.size() * sizeof(float));
  float* d = alloc_f(v.size());
  KGX_HIP(hipMemcpy(d, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
  uploads_.emplace_back(d, v.size() * sizeof(float));
  return d;
}

void Net::upload_mm(RowMM& mm, const std::vector<float>& w, const std::vector<float>& b) {
  if (w.size() != (size_t)mm.IC * mm.OC || b.size() != (size_t)mm.OC)
    throw std::runtime_error("internal: row matmul and bias sizes differ");
  std::vector<float> wb((w.size() + b.size() + 3) / 4 * 4, 0.f);
  std::copy(w.begin(), w.end(), wb.begin());
  std::copy(b.begin(), b.end(), wb.begin() + w.size());
  mm.W = upload_f(wb);
  mm.bias = mm.W + w.size();
}

const void* Net::upload_t(const std::vector<float>& v) {
  if (prec_ == PREC_F32) return upload_f(v);
  if (primary_) return take_upload(v.size() * 2);
  std::vector<uint16_t> h(v.size());
  for (size_t k = 0; k < v.size(); k++) h[k] = prec_ == PREC_F16 ? f32_to_f16_bits(v[k]) : f32_to_bf16_bits(v[k]);
  void* d = alloc_bytes(h.size() * 2);
  KGX_HIP(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice));
  uploads_.emplace_back(d, h.size() * 2);
  return d;
}

RowProg Net::row_prog_base() const {
  RowProg p;
  p.mask = mask_;
  p.area = area_;
  p.s1 = s1_;
  p.s2 = s2_;
  return p;
}

Prologue Net::bn_pro(const BNDesc& bn, int act, const float* prebias, int ld_prebias) {
  Prologue p;
  p.scale = upload_f(bn.scale);
  p.bias = upload_f(bn.bias);
  p.prebias = prebias;
  p.ld_prebias = ld_prebias;
  p.act = act;
  p.mask = mask_;
  return p;
}

Emit Net::bn_emit(const BNDesc& bn, int act, void* out, int ld) {
  Emit e;
  e.scale = upload_f(bn.scale);
  e.bias = upload_f(bn.bias);
  e.act = act;
  e.mask = mask_;
  e.out = out;
  e.ld = ld;
  return e;
}

void* Net::consume(int depth, const BNDesc& bn, int act, const void** lo) {
  StreamState& st = ss_[depth];
  if (!st.producer || st.producer->emit.scale) throw std::runtime_error("internal: stream activation has no producer");
  void* buf = st.act[st.flip];
  st.producer->emit = bn_emit(bn, act, buf, st.c);
  if (lo) {
    // Sized like the stream's high-plane buffers: for the widest block of the stream, not this one.
    if (!st.act_lo[st.flip]) st.act_lo[st.flip] = alloc_bytes((size_t)max_batch_ * HW * stream_c_[depth] * tsize());
    st.producer->emit.out_lo = st.act_lo[st.flip];
    *lo = st.act_lo[st.flip];
  }
  st.flip ^= 1;
  st.producer.reset();
  return buf;
}

static bool is_1x1(const ConvDesc& d) { return d.ky == 1 && d.kx == 1 && d.dy == 1 && d.dx == 1; }

bool Net::exit_fits(const BlockDesc& b, int c) const {
  const ConvDesc& ex = b.final_conv;
  return junctions_ && prec_ != PREC_F32 && conv_mode_ == CONV_IGEMM && is_1x1(ex) && c == kJunctionOuter &&
         ex.ic == kJunctionInner && ex.oc == kJunctionOuter && b.regular.oc == kJunctionInner &&
         ex.w.size() == (size_t)kJunctionInner * kJunctionOuter;
}

bool Net::stem_junction_fits(const ModelDesc& m, const ConvOut& stem_out) const {
  const ConvDesc& st = m.stem;
  if (!junctions_ || prec_ == PREC_F32 || conv_mode_ != CONV_IGEMM || m.blocks.empty()) return false;
  const BlockDesc& b = m.blocks[0];
  const ConvDesc& en = b.regular;
  return st.ky == 3 && st.kx == 3 && st.dy == 1 && st.dx == 1 && st.oc == kJunctionOuter && st.ic >= 1 &&
         st.ic <= 32 && st.w.size() == (size_t)kJunctionOuter * st.ic * 9 && igemm_eligible(st, true, 0, stem_out) &&
         stem_out.colbias && b.kind == BLOCK_NBT && is_1x1(en) && en.ic == kJunctionOuter &&
         en.oc == kJunctionInner && en.w.size() == (size_t)kJunctionInner * kJunctionOuter;
}

bool Net::junction_fits(const BlockDesc& b, const BlockDesc& next, int c) const {
  const ConvDesc& en = next.regular;
  return exit_fits(b, c) && next.kind == BLOCK_NBT && is_1x1(en) && en.ic == kJunctionOuter &&
         en.oc == kJunctionInner && en.w.size() == (size_t)kJunctionInner * kJunctionOuter;
}

std::shared_ptr<ConvOut> Net::emit_junction(const PendingExit& p, const ConvDesc& entry, const ConvOut& entry_o) {
  std::vector<float> w;
  const int eoc = entry.oc;
  if (p.stem) stem_junction_pack_weights(p.conv->w.data(), p.conv->ic, entry.w.data(), eoc, prec_, w);
  else junction_pack_weights(p.conv->w.data(), entry.w.data(), eoc, prec_, w);
  const void* dW = upload_t(w);
  const std::shared_ptr<ConvOut> eo = p.out, no = std::make_shared<ConvOut>(entry_o);
  const int prec = prec_, ldx = p.ldx;
  const void *x = p.x, *x_lo = p.x_lo;
  const double ts = (double)tsize();
  Op op;
  if (p.stem) {
    op.launch = [=](hipStream_t s, int B) { launch_stem_junction(prec, x, ldx, dW, *eo, *no, B, s); };
    op.cls = "stem_junction";
    op.flops_row = 2.0 * HW * (9.0 * p.conv->ic * kJunctionOuter + (double)kJunctionOuter * eoc);
    // The packed input planes, the trunk written, the entry's float output written.
    op.bytes_row = (double)HW * (ldx * ts + 4.0 * kJunctionOuter + 4.0 * eoc);
    op.bytes_fixed = (9.0 * p.conv->ic + 2.0 * eoc) * kJunctionOuter * ts;
  } else {
    op.launch = [=](hipStream_t s, int B) { launch_junction(prec, x, x_lo, ldx, dW, *eo, *no, eoc, B, s); };
    const bool head = eoc == kJunctionHead;
    op.cls = head ? "head_junction" : "conv1x1_junction";
    op.flops_row = 2.0 * HW * (kJunctionInner + eoc) * kJunctionOuter;
    // The exit's split operand, the trunk read and (but where it ends, before the heads) written, the entry's float
    // output written (its emission is counted through `out`).
    op.bytes_row = (double)HW * (2.0 * kJunctionInner * ts + (head ? 4.0 : 8.0) * kJunctionOuter + 4.0 * eoc);
    op.bytes_fixed = 2.0 * (kJunctionInner + eoc) * kJunctionOuter * ts;
  }
  op.out = no;
  op.out_c = eoc;
  op.w = dW;
  op.w_bytes = w.size() * tsize();
  op.pf_sink = no;
  ops_.push_back(op);
  return no;
}

bool Net::split_1x1(const ConvDesc& c, int ldx, const ConvOut& o) const {
  return prec_ != PREC_F32 && c.ky == 1 && c.kx == 1 && c.dy == 1 && c.dx == 1 && igemm_eligible(c, false, ldx, o);
}

// Workspace needs of a block stack with `c` channels at nesting depth `depth`.
void Net::scan(const std::vector<BlockDesc>& blocks, int c, int depth) {
  for (const BlockDesc& b : blocks) {
    switch (b.kind) {
      case BLOCK_RES:
        mid_c_ = std::max(mid_c_, b.regular.oc);
        break;
      case BLOCK_GPOOL:
        tmp_c_ = std::max(tmp_c_, b.regular.oc + b.gconv.oc);
        mid_c_ = std::max(mid_c_, b.regular.oc);
        gb_c_ = std::max(gb_c_, b.regular.oc);
        break;
      case BLOCK_NBT:
        if ((int)stream_c_.size() <= depth + 1) stream_c_.resize(depth + 2, 0);
        stream_c_[depth + 1] = std::max(stream_c_[depth + 1], b.regular.oc);
        scan(b.inner, b.regular.oc, depth + 1);
        break;
      case BLOCK_ATTN:
        nrm_c_ = std::max(nrm_c_, c);
        qkv_c_ = std::max(qkv_c_, b.q.oc + b.k.oc + b.v.oc);
        ao_c_ = std::max(ao_c_, b.heads * b.dv);
        break;
      case BLOCK_FFN:
        nrm_c_ = std::max(nrm_c_, c);
        if (b.swiglu && b.ffn_c % 16) u_c_ = std::max(u_c_, 2 * b.ffn_c);  // the unfused SwiGLU's float u
        h_c_ = std::max(h_c_, b.ffn_c);
        break;
    }
  }
}

// conv(x) into `o`. 3x3 undilated convs run as Winograd (crates/katago-nn-burn/src/wino/ext.rs:324-437): with
// F(2x2,3x3) as an input transform plus one kernel for the 16 point GEMMs and the output transform, with
// F(4x4,3x3) as input transform, 36 batched MFMA GEMMs and output transform. 1x1 convs over NHWC rows are one MFMA
// GEMM (wino/ext.rs:278-321); anything else is a direct convolution.
bool Net::igemm_eligible(const ConvDesc& c, bool nchw, int ldx, const ConvOut& o) const {
  const bool k3 = c.ky == 3 && c.kx == 3 && c.dy == 1 && c.dx == 1, k1 = c.ky == 1 && c.kx == 1;
  const bool strides4 = (!o.y || o.ldy % 4 == 0) && (!o.yt || o.ldyt % 4 == 0) &&
                        (!o.colbias || o.ld_colbias % 4 == 0) && (!o.emit.scale || o.emit.ld % 4 == 0);
  // (The network input is packed by input_prep_kernel, up to 32 planes.)
  return conv_mode_ == CONV_IGEMM && (k3 || k1) && c.oc % 4 == 0 && strides4 &&
         (nchw ? c.ic <= 32 : c.ic % 8 == 0 && ldx % 8 == 0);
}

// The network input planes packed once into compute-type NHWC rows of icin = round_up(ic, 8) channels (0/1 planes
// are exact in 16 bits), with the board statistics and the stem's global bias in the same launch.
const void* Net::emit_input_pack(const ConvDesc& c, const void* x, int& icin) {
  const int prec = prec_, ic = c.ic, ld = round_up(ic, 8);
  icin = ld;
  void* packed = alloc_bytes((size_t)max_batch_ * HW * ld * tsize());
  const float* bin = (const float*)x;
  float *mask = mask_, *area = area_, *s1 = s1_, *s2 = s2_;
  Op pk;
  const InputGlobal gl = stem_glob_;
  pk.launch = [=](hipStream_t s, int B) { launch_input_prep(prec, bin, ic, packed, ld, mask, area, s1, s2, B, s, gl); };
  pk.cls = "input_prep";
  pk.bytes_row = (double)HW * ic * 4 + (double)HW * ld * tsize() + HW * 4.0;
  ops_.push_back(pk);
  return packed;
}

std::shared_ptr<ConvOut> Net::emit_conv(const ConvDesc& c, const void* x, int ldx, bool nchw, const ConvOut& o,
                                        const void* x_lo) {
  const int prec = prec_;
  const double ts = (double)tsize();
  auto out = std::make_shared<ConvOut>(o);
  const bool split = x_lo != nullptr;
  if (split && !(!nchw && c.ky == 1 && c.kx == 1 && igemm_eligible(c, nchw, ldx, o)))
    throw std::runtime_error("internal: split operands for implicit-GEMM 1x1 convolutions only");
  const double in_bytes = (double)HW * c.ic * (nchw ? 4.0 : ts);
  // (A convolution with pooling partials stores only its regular channels.)
  const double out_bytes = (double)HW * (c.oc - (o.pool.psum ? o.pool.C : 0)) *
                           ((o.y ? 4.0 : 0.0) * (o.accumulate ? 2 : 1) + (o.yt ? ts : 0.0));
  const int ic = c.ic, oc = c.oc;
  const bool k3 = c.ky == 3 && c.kx == 3 && c.dy == 1 && c.dx == 1;
  if (igemm_eligible(c, nchw, ldx, o)) {
    const int ks = k3 ? 3 : 1;
    const void* xin = x;
    int ldin = ldx, icin = ic;
    if (nchw) {
      xin = emit_input_pack(c, x, icin);
      ldin = icin;
    }
    const int icp = conv_igemm_icp(ks, icin, oc, split), taps = ks * ks;
    // Filters over the (zero-padded) input channels icin, then packed per output tile (split: high and low planes).
    std::vector<float> wi((size_t)oc * icin * taps, 0.f), w;
    for (int oo = 0; oo < oc; oo++)
      for (int i = 0; i < ic; i++)
        for (int t = 0; t < taps; t++) wi[((size_t)oo * icin + i) * taps + t] = c.w[((size_t)oo * ic + i) * taps + t];
    conv_igemm_pack_weights(ks, wi.data(), oc, icin, w, split, prec);
    const void* dW = upload_t(w);
    Op op;
    op.launch = [=](hipStream_t s, int B) {
      launch_conv_igemm(prec, ks, xin, ldin, icin, dW, icp, oc, *out, B, s, x_lo);
    };
    op.cls = conv_igemm_class(ks, icin, oc, split);
    op.flops_row = 2.0 * HW * ic * oc * taps;
    op.bytes_row = (double)HW * icin * ts * (split ? 2 : 1) + out_bytes;
    op.bytes_fixed = (double)taps * ic * oc * ts * (split ? 2 : 1);
    op.out = out;
    op.out_c = oc;
    op.w = dW;
    op.w_bytes = w.size() * tsize();
    op.pf_sink = out;
    ops_.push_back(op);
    return out;
  }
  if (k3) {
    const int tm = wino_tm_, np = wino_points(tm), nt = wino_tiles(tm);
    const int icp = round_up(c.ic, 32), ocp = round_up(c.oc, 64);
    std::vector<float> U((size_t)np * ocp * icp);
    wino_filter_host(tm, c.w.data(), c.oc, c.ic, ocp, icp, U.data());
    const void* dU = upload_t(U);
    wino_v_elems_ = std::max(wino_v_elems_, (size_t)t_pad(max_batch_) * np * icp);
    Op in;
    in.launch = [=](hipStream_t s, int B) { launch_wino_in(prec, tm, x, ldx, nchw, wino_v_, B, ic, icp, s); };
    in.cls = "wino_in";
    in.bytes_row = in_bytes + (double)np * nt * ic * ts;
    ops_.push_back(in);
    if (tm == 2) {
      Op fu;
      fu.launch = [=](hipStream_t s, int B) { launch_wino2_fused(prec, wino_v_, dU, t_pad(B), icp, ocp, oc, *out, B, s); };
      fu.cls = "wino_gemm";
      fu.flops_row = 2.0 * np * nt * ic * oc;
      fu.bytes_row = (double)np * nt * ic * ts + out_bytes;
      fu.bytes_fixed = (double)np * ic * oc * ts;
      fu.out = out;
      fu.out_c = oc;
      ops_.push_back(fu);
      return out;
    }
    wino_m_elems_ = std::max(wino_m_elems_, (size_t)t_pad(max_batch_) * np * ocp);
    Op gm;
    gm.launch = [=](hipStream_t s, int B) {
      GemmArgs g;
      g.A = wino_v_; g.lda = (long)np * icp; g.sA = icp;
      g.Bt = dU; g.ldb = icp; g.sB = (long)ocp * icp;
      g.out.y = wino_m_; g.out.ldy = np * ocp; g.sC = ocp;
      g.M = B * nt; g.N = ocp; g.K = icp; g.Z = np;
      launch_gemm(prec, g, s);
    };
    gm.cls = "wino_gemm";
    gm.flops_row = 2.0 * np * nt * ic * oc;
    gm.bytes_row = (double)np * nt * ic * ts + (double)np * nt * oc * 4;
    gm.bytes_fixed = (double)np * ic * oc * ts;
    ops_.push_back(gm);
    Op wo;
    wo.launch = [=](hipStream_t s, int B) { launch_wino_out(prec, tm, wino_m_, ocp, oc, *out, B, s); };
    wo.cls = "wino_out";
    wo.bytes_row = (double)np * nt * oc * 4 + out_bytes;
    wo.out = out;
    wo.out_c = oc;
    ops_.push_back(wo);
    return out;
  }
  const int vec = prec == PREC_F32 ? 4 : 8;
  if (c.ky == 1 && c.kx == 1 && !nchw && c.ic % vec == 0 && ldx % vec == 0) {
    const void* dW = upload_t(c.w);  // [oc][ic] is already the B^T layout
    Op gm;
    gm.launch = [=](hipStream_t s, int B) {
      GemmArgs g;
      g.A = x; g.lda = ldx;
      g.Bt = dW; g.ldb = ic;
      g.out = *out;
      g.M = B * HW; g.N = oc; g.K = ic;
      launch_gemm(prec, g, s);
    };
    gm.cls = "gemm_1x1";
    gm.flops_row = 2.0 * HW * ic * oc;
    gm.bytes_row = in_bytes + out_bytes;
    gm.bytes_fixed = (double)ic * oc * ts;
    gm.out = out;
    gm.out_c = oc;
    ops_.push_back(gm);
    return out;
  }
  // [oc][ic][ky][kx] -> [ic][ky][kx][oc]
  std::vector<float> w((size_t)c.ic * c.ky * c.kx * c.oc);
  for (int oo = 0; oo < c.oc; oo++)
    for (int i = 0; i < c.ic; i++)
      for (int a = 0; a < c.ky; a++)
        for (int b = 0; b < c.kx; b++)
          w[(((size_t)i * c.ky + a) * c.kx + b) * c.oc + oo] = c.w[(((size_t)oo * c.ic + i) * c.ky + a) * c.kx + b];
  const float* dW = upload_f(w);
  const int ky = c.ky, kx = c.kx, dy = c.dy, dx = c.dx;
  Op op;
  op.launch = [=](hipStream_t s, int B) { launch_conv_direct(prec, x, ldx, nchw, ic, dW, oc, ky, kx, dy, dx, *out, B, s); };
  op.cls = "conv_direct";
  op.flops_row = 2.0 * HW * ic * oc * ky * kx;
  op.bytes_row = in_bytes + out_bytes;
  op.out = out;
  op.out_c = oc;
  ops_.push_back(op);
  return out;
}

std::shared_ptr<ConvOut> Net::emit_token_gemm(const void* A, int lda, const void* Bt, int N, int K, const ConvOut& o,
                                              const char* cls, bool glu, const QkvEpi& qkv, int yt_act) {
  const int prec = prec_;
  auto out = std::make_shared<ConvOut>(o);
  Op op;
  op.launch = [=](hipStream_t s, int B) {
    GemmArgs g;
    g.A = A; g.lda = lda;
    g.Bt = Bt; g.ldb = K;
    g.out = *out;
    g.M = B * HW; g.N = N; g.K = K;
    g.glu = glu;
    g.qkv = qkv;
    g.yt_act = yt_act;
    launch_gemm(prec, g, s);
  };
  op.cls = cls;
  const double ts = (double)tsize();
  op.flops_row = 2.0 * HW * K * N;
  op.bytes_row = (double)HW * K * ts +
                 (double)HW * N * ((o.y ? 4.0 : 0.0) * (o.accumulate ? 2 : 1) + (o.yt ? (glu ? ts / 2 : ts) : 0.0) +
                                   (o.emit.scale ? ts : 0.0));
  op.bytes_fixed = (double)K * N * ts;
  op.out = out;
  op.out_c = N;
  ops_.push_back(op);
  return out;
}

// TransformerAttentionBlock (bin2onnx.py:1357-1421): RMSNorm, fused q|k|v projection (RoPE-permuted q and k
// columns, bin2onnx.py:1369-1374), attention with RoPE on load, out projection * mask + residual.
void Net::emit_attention(const BlockDesc& b, int depth) {
  const int prec = prec_;
  float* x = ss_[depth].x;
  const int c = ss_[depth].c;
  const int H = b.heads, KV = b.kv_heads, dq = b.dq, dv = b.dv;
  if (dq != dv) throw std::runtime_error(b.name + ": attention with qHeadDim != vHeadDim is not supported");
  const int nq = H * dq, nk = KV * dq, nv = KV * dv, nqkv = nq + nk + nv;
  // B^T rows: output features; per head, RoPE pairs (2p, 2p+1) move to (p, p + dq/2).
  std::vector<float> w((size_t)nqkv * c);
  auto col_of = [&](int j) {
    if (!b.rope) return j;
    const int h = j / dq, r = j - h * dq, half = dq / 2;
    return h * dq + (r < half ? 2 * r : 2 * (r - half) + 1);
  };
  for (int j = 0; j < nq; j++)
    for (int k = 0; k < c; k++) w[(size_t)j * c + k] = b.q.w[(size_t)k * nq + col_of(j)];
  for (int j = 0; j < nk; j++)
    for (int k = 0; k < c; k++) w[(size_t)(nq + j) * c + k] = b.k.w[(size_t)k * nk + col_of(j)];
  for (int j = 0; j < nv; j++)
    for (int k = 0; k < c; k++) w[(size_t)(nq + nk + j) * c + k] = b.v.w[(size_t)k * nv + j];
  const void* dWqkv = upload_t(w);
  std::vector<float> wo((size_t)c * H * dv);
  for (int o = 0; o < c; o++)
    for (int k = 0; k < H * dv; k++) wo[(size_t)o * H * dv + k] = b.o.w[(size_t)k * c + o];
  const void* dWo = upload_t(wo);
  // RoPE tables [tables][HW][dq/2], float, as computeRopeCosSin (bin2onnx.py:449-485).
  const float* dcos = nullptr;
  const float* dsin = nullptr;
  int ntab = 0;
  if (b.rope) {
    const int pairs = dq / 2;
    ntab = b.learnable_rope ? KV : 1;
    std::vector<float> cs((size_t)ntab * HW * pairs), sn(cs.size());
    for (int t = 0; t < ntab; t++)
      for (int p = 0; p < pairs; p++)
        for (int y = 0; y < POS; y++)
          for (int xx = 0; xx < POS; xx++) {
            float ang;
            if (b.learnable_rope) {
              const float fx = b.rope_freqs[((size_t)t * pairs + p) * 2], fy = b.rope_freqs[((size_t)t * pairs + p) * 2 + 1];
              ang = (float)xx * fx + (float)y * fy;
            } else {
              const int per_dim = pairs / 2;
              const int padj = p < per_dim ? p : p - per_dim;
              const float expo = (float)(2 * padj) / (float)(dq / 2);
              const float powv = (float)std::pow((double)b.rope_theta, (double)expo);
              const float freq = 1.0f / powv;
              ang = (p < per_dim ? (float)y : (float)xx) * freq;
            }
            const size_t idx = ((size_t)t * HW + y * POS + xx) * pairs + p;
            cs[idx] = (float)std::cos((double)ang);
            sn[idx] = (float)std::sin((double)ang);
          }
    dcos = upload_f(cs);
    dsin = upload_f(sn);
  }
  const float* lnw = upload_f(b.ln_w);
  const float eps = b.ln_eps;
  void* nrm = nrm_;
  const float* mask = mask_;
  Op rn;
  const int rn_n = res_n_, rn_k = res_k_;
  rn.launch = [=](hipStream_t s, int B) {
    const int region = rn_n ? gemm_row_tile(prec, B * HW, rn_n, rn_k) : 0;
    launch_rmsnorm_tok(prec, x, c, c, lnw, eps, mask, nrm, c, B * HW, s, region);
  };
  rn.cls = "rmsnorm";
  rn.bytes_row = (double)HW * c * (4 + tsize());
  ops_.push_back(rn);
  // The projection's epilogue applies RoPE to the query and key heads and the 1/sqrt(dq) scale to the queries,
  // so attention reads them ready to use.
  ConvOut oq;
  oq.yt = qkv_;
  oq.ldyt = nqkv;
  QkvEpi qe;
  qe.cos = dcos; qe.sin = dsin; qe.dq = dq; qe.nq = nq; qe.nk = nk; qe.H = H; qe.KV = KV; qe.tables = ntab;
  qe.qscale = 1.0f / std::sqrt((float)dq);
  emit_token_gemm(nrm_, c, dWqkv, nqkv, c, oq, "token_gemm_qkv", false, qe);
  void* qkv = qkv_;
  void* ao = ao_;
  Op at;
  at.launch = [=](hipStream_t s, int B) {
    AttnArgs a;
    a.qkv = qkv; a.ldq = nqkv; a.q_off = 0; a.k_off = nq; a.v_off = nq + nk;
    a.H = H; a.KV = KV; a.dq = dq; a.dv = dv;
    a.scale = 1.f; a.mask = mask; a.out = ao; a.ldo = H * dv;
    launch_attention(prec, a, B, s);
  };
  at.cls = "attention";
  at.flops_row = 2.0 * H * HW * HW * (dq + dv);
  at.bytes_row = (double)HW * nqkv * tsize() + (double)HW * H * dv * tsize();
  ops_.push_back(at);
  ConvOut oo;
  oo.y = x; oo.ldy = c; oo.accumulate = true; oo.rowmask = mask;
  ss_[depth].producer = emit_token_gemm(ao_, H * dv, dWo, c, H * dv, oo, "token_gemm_out");
  res_n_ = c;
  res_k_ = H * dv;
}

// TransformerFFNBlock (bin2onnx.py:1423-1438): RMSNorm, linear1 (| gate), SiLU(l1) * gate (the plain FFN, which
// the reference rejects, as mish(l1)), linear2 * mask + residual.
void Net::emit_ffn(const BlockDesc& b, int depth) {
  const int prec = prec_;
  float* x = ss_[depth].x;
  const int c = ss_[depth].c;
  const int F = b.ffn_c, Fu = b.swiglu ? 2 * F : F;
  // The activation runs in the first GEMM's epilogue: SwiGLU through its gated output, whose B^T rows alternate
  // 16 value features and the 16 matching gate features (F % 16 == 0; otherwise u = [value | gate] goes through
  // the separate activation kernel); mish as the activation of its compute-type output.
  const bool fused = !b.swiglu || F % 16 == 0;
  auto row_of = [&](int f, bool gate) {
    if (!b.swiglu) return f;
    if (!fused) return gate ? F + f : f;
    return (f / 16) * 32 + (gate ? 16 : 0) + f % 16;
  };
  std::vector<float> w1((size_t)Fu * c);
  for (int f = 0; f < F; f++)
    for (int k = 0; k < c; k++) {
      w1[(size_t)row_of(f, false) * c + k] = b.l1.w[(size_t)k * F + f];
      if (b.swiglu) w1[(size_t)row_of(f, true) * c + k] = b.lg.w[(size_t)k * F + f];
    }
  const void* dW1 = upload_t(w1);
  std::vector<float> w2((size_t)c * F);
  for (int o = 0; o < c; o++)
    for (int f = 0; f < F; f++) w2[(size_t)o * F + f] = b.l2.w[(size_t)f * c + o];
  const void* dW2 = upload_t(w2);
  const float* lnw = upload_f(b.ln_w);
  const float eps = b.ln_eps;
  void* nrm = nrm_;
  const float* mask = mask_;
  Op rn;
  const int rn_n = res_n_, rn_k = res_k_;
  rn.launch = [=](hipStream_t s, int B) {
    const int region = rn_n ? gemm_row_tile(prec, B * HW, rn_n, rn_k) : 0;
    launch_rmsnorm_tok(prec, x, c, c, lnw, eps, mask, nrm, c, B * HW, s, region);
  };
  rn.cls = "rmsnorm";
  rn.bytes_row = (double)HW * c * (4 + tsize());
  ops_.push_back(rn);
  ConvOut o1;
  if (fused && b.swiglu) {
    o1.yt = h_;
    o1.ldyt = F;
    emit_token_gemm(nrm_, c, dW1, Fu, c, o1, "token_gemm_ffn1", true);
  } else if (fused) {
    o1.yt = h_;
    o1.ldyt = F;
    emit_token_gemm(nrm_, c, dW1, Fu, c, o1, "token_gemm_ffn1", false, QkvEpi(), ACT_MISH);
  } else {
    o1.y = u_;
    o1.ldy = Fu;
    emit_token_gemm(nrm_, c, dW1, Fu, c, o1, "token_gemm_ffn1");
    float* u = u_;
    void* h = h_;
    const bool gated = b.swiglu;
    Op fa;
    fa.launch = [=](hipStream_t s, int B) { launch_ffn_act(prec, u, Fu, F, gated, h, F, B * HW, s); };
    fa.cls = "ffn_act";
    fa.bytes_row = (double)HW * Fu * 4 + (double)HW * F * tsize();
    ops_.push_back(fa);
  }
  ConvOut o2;
  o2.y = x; o2.ldy = c; o2.accumulate = true; o2.rowmask = mask;
  ss_[depth].producer = emit_token_gemm(h_, F, dW2, c, F, o2, "token_gemm_ffn2");
  res_n_ = c;
  res_k_ = F;
}

void Net::emit_stack(const std::vector<BlockDesc>& blocks, int depth) {
  const int prec = prec_;
  for (size_t bi = 0; bi < blocks.size(); bi++) {
    const BlockDesc& b = blocks[bi];
    float* x = ss_[depth].x;
    const int c = ss_[depth].c;
    ConvOut res;  // the block's residual add into its stream
    res.y = x;
    res.ldy = c;
    res.accumulate = true;
    if (b.kind != BLOCK_ATTN && b.kind != BLOCK_FFN) res_n_ = res_k_ = 0;
    switch (b.kind) {
      case BLOCK_RES: {
        // x += conv2(bnact(conv1(bnact(x)))) (bin2onnx.py:1243-1249); conv1 writes only conv2's activation.
        const int cm = b.regular.oc;
        const void* a = consume(depth, b.pre_bn, b.pre_act);
        ConvOut o1;
        o1.emit = bn_emit(b.mid_bn, b.mid_act, mid_, cm);
        emit_conv(b.regular, a, c, false, o1);
        ss_[depth].producer = emit_conv(b.final_conv, mid_, cm, false, res);
        break;
      }
      case BLOCK_GPOOL: {
        // regular | gpool convs share their input: one convolution with both filters (bin2onnx.py:1250-1261).
        const int cr = b.regular.oc, cg = b.gconv.oc, ct = cr + cg;
        ConvDesc both = b.regular;
        both.oc = ct;
        both.w.insert(both.w.end(), b.gconv.w.begin(), b.gconv.w.end());
        if (b.regular.ky != b.gconv.ky || b.regular.kx != b.gconv.kx || b.regular.dy != b.gconv.dy || b.regular.dx != b.gconv.dx)
          throw std::runtime_error(b.name + ": regular and gpool convolutions differ in shape");
        const void* a = consume(depth, b.pre_bn, b.pre_act);
        ConvOut o1;
        o1.y = tmp_;
        o1.ldy = ct;
        // The pooled branch's batch norm and activation, and on the implicit-GEMM path its board pooling as
        // partials of the conv's tiles (PoolPart), so that the row program reads at most three partials per board
        // instead of its 361 rows, and the branch's float output is not stored. The branches' filters are then
        // interleaved per column tile (cr / tiles regular, then cg / tiles pooled channels), which spreads the
        // pooling over all workgroups of the conv's single wave (b18c384nbt: 48 + 16 of 64 columns per tile).
        const float* gsc = upload_f(b.gbn.scale);
        const float* gbi = upload_f(b.gbn.bias);
        long long* psum = nullptr;
        float* pmax = nullptr;
        const int pbn = conv_igemm_pool_cols(both.ky, c, ct), ptiles = pbn ? ct / pbn : 0;
        const int pgroups = ptiles ? cg / ptiles / 4 : 0;  // pooled channel groups per tile: a power of two <= 16
        if (igemm_eligible(both, false, c, o1) && pbn && ct % pbn == 0 && cr % (4 * ptiles) == 0 &&
            cg % (4 * ptiles) == 0 && pgroups > 0 && pgroups <= 16 && (pgroups & (pgroups - 1)) == 0 &&
            conv_igemm_tile_rows(both.ky, c, ct) == 192) {
          const int rpt = cr / ptiles, gpt = cg / ptiles;
          const size_t fl = both.w.size() / ct;  // floats per output channel
          std::vector<float> w;
          w.reserve(both.w.size());
          for (int t = 0; t < ptiles; t++) {
            const auto reg = both.w.begin() + (size_t)t * rpt * fl;
            const auto gp = both.w.begin() + ((size_t)cr + (size_t)t * gpt) * fl;
            w.insert(w.end(), reg, reg + (size_t)rpt * fl);
            w.insert(w.end(), gp, gp + (size_t)gpt * fl);
          }
          both.w.swap(w);
          const size_t n = ((size_t)max_batch_ * HW + 191) / 192 * 2 * cg;
          psum = (long long*)alloc_bytes(n * sizeof(long long));
          pmax = alloc_f(n);
          o1.pool.psum = psum;
          o1.pool.pmax = pmax;
          o1.pool.scale = gsc;
          o1.pool.bias = gbi;
          o1.pool.act = b.gact;
          o1.pool.mask = mask_;
          o1.pool.rpt = rpt;
          o1.pool.C = cg;
        }
        emit_conv(both, a, c, false, o1);
        // Pooling of the gpool branch (after its batch norm and activation) and the matmul to the bias of the
        // regular branch, one workgroup per row.
        float* tmp = tmp_;
        float* gb = gb_;
        RowProg rp = row_prog_base();
        rp.npool = 1;
        rp.pool[0].x = tmp; rp.pool[0].ldx = ct; rp.pool[0].coff = cr; rp.pool[0].C = cg;
        rp.pool[0].scale = gsc; rp.pool[0].bias = gbi; rp.pool[0].act = b.gact;
        rp.pool[0].dst = 0;
        if (psum) {
          rp.pool[0].psum = psum;
          rp.pool[0].pmax = pmax;
          rp.pool[0].ppt = 192;
        }
        rp.nmm = 1;
        rp.mm[0].src = 0; rp.mm[0].IC = 3 * cg; rp.mm[0].OC = cr; rp.mm[0].W = upload_f(b.gmul.w);
        rp.mm[0].out = gb; rp.mm[0].ldout = cr;
        rp.lds_floats = 3 * cg;
        rp.splits = std::max(1, std::min(8, cr / 64));
        // The mid activation adds the pooled bias per (row, channel) before its batch norm. With 16-bit compute
        // types the row program's workgroups emit it for their share of the channels (the bias stays in LDS),
        // as many shares per row as fit up to eight (b18c384nbt: 8 x 24 channels, 0.5 % faster end to end than
        // 3 x 64 with the emission or than a separate bias_act launch); otherwise a bias_act launch follows.
        const Emit me = bn_emit(b.mid_bn, b.mid_act, mid_, cr);
        int fsplits = 0;
        for (int sp = 8; sp >= 1 && !fsplits; sp--)
          if (row_emit_fits(cr, sp)) fsplits = sp;
        const bool fuse = prec != PREC_F32 && fsplits > 0 && ct % 4 == 0 && me.ld % 8 == 0;
        if (fuse) {
          rp.splits = fsplits;
          rp.mm[0].out = nullptr;
          rp.mm[0].dst = 3 * cg;
          rp.lds_floats = 3 * cg + cr;
          rp.emit.x = tmp; rp.emit.ldx = ct;
          rp.emit.scale = me.scale; rp.emit.bias = me.bias; rp.emit.act = me.act;
          rp.emit.out = me.out; rp.emit.ldo = me.ld; rp.emit.prec = prec;
          // Each workgroup's share of the matmul's weights staged in LDS with the program's first loads, so the
          // matmul after the pooling waits for no memory (17.7 -> 12.x us per row program at b18c384nbt).
          const int share = cr / fsplits;
          const int woff = (rp.lds_floats + 3) / 4 * 4;
          const size_t lds = ((size_t)woff + 3 * cg * share + 2 * 1024 + HW + 2 * cr) * sizeof(float);
          if (cr % fsplits == 0 && share % 4 == 0 && lds <= 64 * 1024) {
            rp.mm[0].wlds = woff;
            rp.mm[0].wcols = share;
            rp.mm[0].w4 = 3 * cg * share / 4;
            rp.lds_floats = woff + 3 * cg * share;
          }
        }
        const int gts = gpool_tile_share(cg, cr);
        if (fuse && psum && gts > 0 && gpool_tile_) {
          // The same arithmetic per 192-pixel tile on the convolutions' XCDs (GpoolTile): a workgroup reads the
          // x rows and writes the emission where the convolutions before and after it write and read them.
          GpoolTile gt;
          gt.psum = psum; gt.pmax = pmax; gt.cg = cg; gt.area = area_; gt.s1 = s1_;
          gt.W = rp.mm[0].W; gt.cr = cr; gt.share = gts;
          gt.x = tmp; gt.ldx = ct; gt.scale = me.scale; gt.bias = me.bias; gt.act = me.act; gt.mask = mask_;
          gt.out = me.out; gt.ldo = me.ld; gt.prec = prec;
          const std::shared_ptr<ConvOut> sink = std::make_shared<ConvOut>();  // the next op's weights (pf)
          Op op;
          op.launch = [=](hipStream_t s, int B) {
            GpoolTile g = gt;
            g.pf = sink->pf;
            g.pf_bytes = sink->pf_bytes;
            launch_gpool_tile(g, B, s);
          };
          op.cls = "gpool_tile";
          op.bytes_row = (double)HW * cr * (4 + tsize());
          op.flops_row = 2.0 * 3 * cg * cr;
          op.w = gt.W;
          op.w_bytes = (size_t)3 * cg * cr * sizeof(float);
          op.pf_sink = sink;
          ops_.push_back(op);
          ss_[depth].producer = emit_conv(b.final_conv, mid_, cr, false, res);
          break;
        }
        Op pool;
        pool.launch = [=](hipStream_t s, int B) { launch_row_prog(rp, B, s); };
        pool.cls = "row_prog_gpool";
        pool.bytes_row = (double)HW * cg * 4 + (fuse ? (double)HW * cr * (4 + tsize()) : 0.0);
        pool.flops_row = 2.0 * 3 * cg * cr;
        ops_.push_back(pool);
        if (!fuse) {
          Op ba;
          ba.launch = [=](hipStream_t s, int B) {
            launch_bias_act(prec, tmp, ct, cr, gb, cr, me.scale, me.bias, me.act, me.mask, me.out, me.ld, B * HW, s);
          };
          ba.cls = "bias_act";
          ba.bytes_row = (double)HW * cr * (4 + tsize());
          ops_.push_back(ba);
        }
        ss_[depth].producer = emit_conv(b.final_conv, mid_, cr, false, res);
        break;
      }
      case BLOCK_NBT: {
        // x += post(bnact(inner(pre(bnact(x))))) (bin2onnx.py:1263-1269)
        // The entry and exit 1x1 convolutions run on split operands on 16-bit handles (only 3x3 convolutions
        // round their operands to 16 bits, as in the reference's f16 mode, backend.rs:399-403).
        const int ci = b.regular.oc;
        StreamState& in = ss_[depth + 1];
        ConvOut o1;
        o1.y = in.x;
        o1.ldy = ci;
        const void* a_lo = nullptr;
        const void* a = consume(depth, b.pre_bn, b.pre_act, split_1x1(b.regular, c, o1) ? &a_lo : nullptr);
        in.c = ci;
        in.producer.reset();
        if (pend_) {
          // The previous block's exit convolution was held back for this entry: one junction launch for both.
          if (pend_->out->emit.out != a || pend_->out->emit.out_lo != a_lo || !a_lo)
            throw std::runtime_error("internal: junction entry does not consume the held exit");
          in.producer = emit_junction(*pend_, b.regular, o1);
          pend_.reset();
        } else {
          in.producer = emit_conv(b.regular, a, c, false, o1, a_lo);
        }
        emit_stack(b.inner, depth + 1);
        // The inner stream ends with this activation: its last producer computes the stream's final value only
        // for the emission, so that sum is not stored.
        const std::shared_ptr<ConvOut> last = ss_[depth + 1].producer;
        const void* a2_lo = nullptr;
        const void* a2 = consume(depth + 1, b.mid_bn, b.mid_act, split_1x1(b.final_conv, ci, res) ? &a2_lo : nullptr);
        if (last) last->y_dead = true;
        const bool to_heads = depth == 0 && bi + 1 == blocks.size() && head_junction_ && exit_fits(b, c);
        if (a2_lo && ((bi + 1 < blocks.size() && junction_fits(b, blocks[bi + 1], c)) || to_heads)) {
          // Held back: the next block's entry convolution joins it (its consume attaches this emission).
          if (pend_) throw std::runtime_error("internal: two exits held back");
          pend_.reset(new PendingExit{&b.final_conv, a2, a2_lo, ci, std::make_shared<ConvOut>(res)});
          ss_[depth].producer = pend_->out;
        } else {
          ss_[depth].producer = emit_conv(b.final_conv, a2, ci, false, res, a2_lo);
        }
        break;
      }
      case BLOCK_ATTN:
        emit_attention(b, depth);
        break;
      case BLOCK_FFN:
        emit_ffn(b, depth);
        break;
    }
  }
}

void Net::build(const ModelDesc& m) {
  const int C = m.trunk_c;
  const size_t Mx = (size_t)max_batch_ * HW;
  nin_ = m.num_input_channels;
  nglob_ = m.num_global;
  nmeta_ = m.num_meta;
  row_len_ = m.row_len();

  if (primary_) {
    // A workspace plan reads and writes the primary's input and output buffers.
    d_bin_ = primary_->d_bin_;
    d_glob_ = primary_->d_glob_;
    d_meta_ = primary_->d_meta_;
    d_out_ = primary_->d_out_;
  } else {
    d_bin_ = alloc_f((size_t)max_batch_ * nin_ * HW);
    d_glob_ = alloc_f((size_t)max_batch_ * nglob_);
    d_meta_ = nmeta_ ? alloc_f((size_t)max_batch_ * nmeta_) : nullptr;
    d_out_ = alloc_f((size_t)max_batch_ * row_len_);
    KGX_HIP(hipMemset(d_bin_, 0, (size_t)max_batch_ * nin_ * HW * 4));
    KGX_HIP(hipMemset(d_glob_, 0, (size_t)max_batch_ * nglob_ * 4));
    if (d_meta_) KGX_HIP(hipMemset(d_meta_, 0, (size_t)max_batch_ * nmeta_ * 4));
  }
  mask_ = alloc_f(Mx);
  area_ = alloc_f(max_batch_);
  s1_ = alloc_f(max_batch_);
  s2_ = alloc_f(max_batch_);

  stream_c_.assign(1, C);
  scan(m.blocks, C, 0);
  trunk_ = alloc_f(Mx * C);
  ss_.assign(stream_c_.size(), StreamState());
  for (size_t d = 0; d < stream_c_.size(); d++) {
    ss_[d].c = stream_c_[d];
    ss_[d].x = d == 0 ? trunk_ : alloc_f(Mx * stream_c_[d]);
    for (int k = 0; k < 2; k++) ss_[d].act[k] = alloc_bytes(Mx * stream_c_[d] * tsize());
  }
  if (tmp_c_) tmp_ = alloc_f(Mx * tmp_c_);
  if (mid_c_) mid_ = alloc_bytes(Mx * mid_c_ * tsize());
  if (gb_c_) gb_ = alloc_f((size_t)max_batch_ * gb_c_);
  if (nrm_c_) nrm_ = alloc_bytes(Mx * nrm_c_ * tsize());
  if (qkv_c_) qkv_ = alloc_bytes(Mx * qkv_c_ * tsize());
  if (ao_c_) ao_ = alloc_bytes(Mx * ao_c_ * tsize());
  if (u_c_) u_ = alloc_f(Mx * u_c_);
  if (h_c_) h_ = alloc_bytes(Mx * h_c_ * tsize());

  // --- Trunk input (bin2onnx.py:1466-1492): mask, stem conv + global (and metadata) bias. ---
  ConvOut stem_out;
  stem_out.y = trunk_;
  stem_out.ldy = C;
  stem_out.ld_colbias = C;
  if (!igemm_eligible(m.stem, true, 0, stem_out)) {  // else the stem's input packing computes the board statistics
    float *bin = d_bin_, *mask = mask_, *area = area_, *s1 = s1_, *s2 = s2_;
    const int nin = nin_;
    Op op;
    op.launch = [=](hipStream_t s, int B) { launch_mask_prep(bin, nin, mask, area, s1, s2, B, s); };
    op.cls = "mask_prep";
    op.bytes_row = HW * 8.0;
    ops_.push_back(op);
  }
  // The stem's per-row bias: global inputs through their matmul, plus the metadata encoder's output
  // (bin2onnx.py:1477-1488), one workgroup per row. Without a metadata encoder, and when the stem packs its
  // input planes (implicit GEMM), the input packing launch computes it (one launch less).
  float* gbias = alloc_f((size_t)max_batch_ * C);
  if (m.meta_version == 0 && nglob_ > 0 && nglob_ <= 32 && igemm_eligible(m.stem, true, 0, stem_out)) {
    stem_glob_.glob = d_glob_; stem_glob_.nglob = nglob_;
    stem_glob_.W = upload_f(m.stem_mm.w); stem_glob_.C = C;
    stem_glob_.out = gbias;
  } else {
    RowProg rp = row_prog_base();
    RowMM& g = rp.mm[rp.nmm++];
    g.gin = d_glob_; g.ldgin = nglob_; g.IC = nglob_; g.OC = C; g.W = upload_f(m.stem_mm.w);
    g.out = gbias; g.ldout = C;
    double flops = 2.0 * nglob_ * C;
    if (m.meta_version > 0) {
      const int h1 = m.meta1.oc, h2 = m.meta2.oc;
      RowMM& a = rp.mm[rp.nmm++];
      a.gin = d_meta_; a.ldgin = nmeta_; a.IC = nmeta_; a.OC = h1; a.W = upload_f(m.meta1.w);
      a.bias = upload_f(m.meta_b1.b); a.act = m.meta_act1; a.dst = 0;
      RowMM& c = rp.mm[rp.nmm++];
      c.src = 0; c.IC = h1; c.OC = h2; c.W = upload_f(m.meta2.w); c.bias = upload_f(m.meta_b2.b);
      c.act = m.meta_act2; c.dst = h1;
      RowMM& d = rp.mm[rp.nmm++];
      d.src = h1; d.IC = h2; d.OC = C; d.W = upload_f(m.meta3.w); d.out = gbias; d.ldout = C; d.accumulate = true;
      rp.lds_floats = h1 + h2;
      flops += 2.0 * ((double)nmeta_ * h1 + (double)h1 * h2 + (double)h2 * C);
    } else {
      rp.splits = std::max(1, std::min(8, C / 64));
    }
    Op op;
    op.launch = [=](hipStream_t s, int B) { launch_row_prog(rp, B, s); };
    op.cls = "row_prog_input";
    op.flops_row = flops;
    ops_.push_back(op);
  }
  stem_out.colbias = gbias;
  if (stem_junction_fits(m, stem_out)) {
    // Held back: the first block's entry convolution joins the stem (its consume attaches the stem's emission).
    int icin = 0;
    const void* packed = emit_input_pack(m.stem, d_bin_, icin);
    pend_.reset(new PendingExit{&m.stem, packed, nullptr, icin, std::make_shared<ConvOut>(stem_out), true});
    ss_[0].producer = pend_->out;
  } else {
    ss_[0].producer = emit_conv(m.stem, d_bin_, 0, true, stem_out);
  }

  // --- Blocks. ---
  // The trunk's last exit may join the heads' p1 | g1 | v1 convolution in one junction launch (16-bit handles, a
  // batch-norm tip, 96 head channels).
  head_junction_ = m.trunk_norm_kind == 0 && m.p1.oc + m.g1.oc + m.v1.oc == kJunctionHead && is_1x1(m.p1) &&
                   is_1x1(m.g1) && is_1x1(m.v1) && m.p1.ic == C && m.g1.ic == C && m.v1.ic == C;
  emit_stack(m.blocks, 0);

  // --- Trunk tip and heads (bin2onnx.py:1489-1531). ---
  for (const ConvDesc* hc : {&m.p1, &m.g1, &m.v1, &m.p2, &m.own})
    if (hc->ky != 1 || hc->kx != 1) throw std::runtime_error(hc->name + ": head convolutions must be 1x1");
  const int cp = m.p1.oc, cg = m.g1.oc, cv = m.v1.oc, nh = cp + cg + cv;
  if (C % 8 != 0) throw std::runtime_error("trunk channels must be a multiple of 8");
  // The head convolutions p1 | g1 | v1 as one 1x1 convolution into H.
  ConvDesc hconv;
  hconv.name = "p1|g1|v1";
  hconv.ky = hconv.kx = 1;
  hconv.ic = C;
  hconv.oc = nh;
  hconv.w.resize((size_t)nh * C);
  std::memcpy(hconv.w.data(), m.p1.w.data(), (size_t)cp * C * 4);
  std::memcpy(hconv.w.data() + (size_t)cp * C, m.g1.w.data(), (size_t)cg * C * 4);
  std::memcpy(hconv.w.data() + (size_t)(cp + cg) * C, m.v1.w.data(), (size_t)cv * C * 4);
  float* H = alloc_f(Mx * nh);
  ConvOut hout;
  hout.y = H;
  hout.ldy = nh;
  const float* head_in = trunk_;
  Prologue tip_pro;
  if (m.trunk_norm_kind == 0 && split_1x1(hconv, C, hout)) {
    // 16-bit handles: the trunk's last producer emits the tip activation as split operands (high and low 16-bit
    // planes) instead of storing the float trunk, and the head convolution runs on them like the nested blocks'
    // 1x1 convolutions (about 22 significant bits per operand, where the float GEMM below has 24).
    const std::shared_ptr<ConvOut> last = ss_[0].producer;
    const void* tip_lo = nullptr;
    const void* tip = consume(0, m.tip_bn, m.tip_act, &tip_lo);
    last->y_dead = true;
    if (pend_) {
      // The trunk's last exit was held back for this convolution: one junction launch for both.
      if (pend_->out != last || !tip_lo || hconv.oc != kJunctionHead)
        throw std::runtime_error("internal: head junction does not consume the held exit");
      emit_junction(*pend_, hconv, hout);
      pend_.reset();
    } else {
      emit_conv(hconv, tip, C, false, hout, tip_lo);
      ops_.back().cls = "head_1x1";
    }
  } else if (m.trunk_norm_kind == 0) {
    tip_pro = bn_pro(m.tip_bn, m.tip_act);
  } else {
    float* tip = alloc_f(Mx * C);
    float* rs = alloc_f(max_batch_);
    const float *gamma = upload_f(m.tip_gamma), *beta = upload_f(m.tip_beta);
    const float eps = m.tip_rms_eps;
    const bool spatial = m.tip_rms_spatial;
    const int act = m.tip_act;
    float *trunk = trunk_, *mask = mask_, *area = area_;
    Op op;
    op.launch = [=](hipStream_t s, int B) { launch_tip_rms(trunk, C, gamma, beta, eps, spatial, act, mask, area, rs, tip, B, s); };
    op.cls = "rmsnorm";
    op.bytes_row = HW * C * 8.0;
    ops_.push_back(op);
    head_in = tip;
  }
  if (pend_) throw std::runtime_error("internal: an exit convolution was held back for no entry");
  if (!(m.trunk_norm_kind == 0 && split_1x1(hconv, C, hout))) {
    // Float operands: float handles, and the trunk-tip RMSNorm's output.
    const float* dWh = upload_f(hconv.w);
    const int prec = PREC_F32;
    Op op;
    op.launch = [=](hipStream_t s, int B) {
      GemmArgs g;
      g.A = head_in; g.lda = C; g.a_float = true; g.pro = tip_pro;
      g.Bt = dWh; g.ldb = C;
      g.out.y = H; g.out.ldy = nh;
      g.M = B * HW; g.N = nh; g.K = C;
      launch_gemm(prec, g, s);
    };
    op.cls = "gemm_1x1";
    op.flops_row = 2.0 * HW * C * nh;
    op.bytes_row = (double)HW * C * 4 + (double)HW * nh * 4;
    ops_.push_back(op);
  }
  const int P = m.P, S = m.S, rl = row_len_;
  float* out = d_out_;
  // Row work of both heads in one launch (bin2onnx.py:1495-1531), as three independent programs that run side by
  // side: g1 pooling -> gpool bias of p1; g1 pooling -> the pass logits; value pooling -> v2 -> value and score
  // outputs. Their small matrices are staged in LDS.
  float* p1b = alloc_f((size_t)max_batch_ * cp);
  {
    const int c2 = m.v2.oc, ph = m.pass1.oc;
    const bool v15 = m.version >= 15;
    RowPool pg;
    pg.x = H; pg.ldx = nh; pg.coff = cp; pg.C = cg;
    pg.scale = upload_f(m.g1_bn.scale); pg.bias = upload_f(m.g1_bn.bias); pg.act = m.g1_act; pg.dst = 0;
    RowPool pv;
    pv.x = H; pv.ldx = nh; pv.coff = cp + cg; pv.C = cv;
    pv.scale = upload_f(m.v1_bn.scale); pv.bias = upload_f(m.v1_bn.bias); pv.act = m.v1_act; pv.value = true;
    pv.dst = 0;
    RowProgs ps;
    ps.n = 3;
    {  // gpool bias of p1
      RowProg& rp = ps.p[0];
      rp = row_prog_base();
      rp.npool = 1; rp.pool[0] = pg; rp.lds_floats = 3 * cg;
      RowMM& gbm = rp.mm[rp.nmm++];
      gbm.src = 0; gbm.IC = 3 * cg; gbm.OC = cp; gbm.W = upload_f(m.gpool_to_bias.w); gbm.out = p1b; gbm.ldout = cp;
    }
    {  // pass logits
      RowProg& rp = ps.p[1];
      rp = row_prog_base();
      rp.npool = 1; rp.pool[0] = pg; rp.lds_floats = 3 * cg;
      if (v15) {
        const int fp = rp.lds_floats; rp.lds_floats += ph;  // pass hidden layer
        RowMM& p1 = rp.mm[rp.nmm++];
        p1.src = 0; p1.IC = 3 * cg; p1.OC = ph; upload_mm(p1, m.pass1.w, m.pass_bias.b);
        p1.act = m.pass_act; p1.dst = fp;
        RowMM& p2 = rp.mm[rp.nmm++];
        p2.src = fp; p2.IC = ph; p2.OC = P; p2.W = upload_f(m.pass2.w);
        p2.out = out + HW; p2.ldout = rl; p2.ostride = HW + 1;
      } else {
        RowMM& p1 = rp.mm[rp.nmm++];
        p1.src = 0; p1.IC = 3 * cg; p1.OC = P; p1.W = upload_f(m.pass1.w);
        p1.out = out + HW; p1.ldout = rl; p1.ostride = HW + 1;
      }
    }
    {  // value and score outputs
      RowProg& rp = ps.p[2];
      rp = row_prog_base();
      rp.npool = 1; rp.pool[0] = pv; rp.lds_floats = 3 * cv;
      const int f2 = rp.lds_floats; rp.lds_floats += c2;  // v2
      RowMM& v2 = rp.mm[rp.nmm++];
      v2.src = 0; v2.IC = 3 * cv; v2.OC = c2; upload_mm(v2, m.v2.w, m.v2_bias.b);
      v2.act = m.v2_act; v2.dst = f2;
      // v3 (3 value logits) and sv3 (S score values) side by side: their outputs are adjacent in the row.
      RowMM& vs = rp.mm[rp.nmm++];
      vs.src = f2; vs.IC = c2; vs.OC = 3 + S;
      std::vector<float> wvs((size_t)c2 * (3 + S)), bvs(3 + S);
      for (int i = 0; i < c2; i++) {
        for (int o = 0; o < 3; o++) wvs[(size_t)i * (3 + S) + o] = m.v3.w[(size_t)i * 3 + o];
        for (int o = 0; o < S; o++) wvs[(size_t)i * (3 + S) + 3 + o] = m.sv3.w[(size_t)i * S + o];
      }
      for (int o = 0; o < 3; o++) bvs[o] = m.v3_bias.b[o];
      for (int o = 0; o < S; o++) bvs[3 + o] = m.sv3_bias.b[o];
      upload_mm(vs, wvs, bvs);
      vs.out = out + P * (HW + 1); vs.ldout = rl;
    }
    for (int k = 0; k < ps.n; k++) row_prog_stage_weights(ps.p[k], 60 * 1024);
    Op op;
    op.launch = [=](hipStream_t s, int B) { launch_row_progs(ps, B, s); };
    op.cls = "row_prog_heads";
    op.bytes_row = (double)HW * (2 * cg + cv) * 4;
    ops_.push_back(op);
  }
  // Spatial policy and ownership.
  {
    HeadSpatialArgs a;
    a.H = H; a.ldh = nh;
    a.p1_off = 0; a.c_p1 = cp; a.p1_bias = p1b;
    a.p1_scale = upload_f(m.p1_bn.scale); a.p1_shift = upload_f(m.p1_bn.bias); a.p1_act = m.p1_act;
    std::vector<float> wp2((size_t)cp * P);
    for (int p = 0; p < P; p++)
      for (int k = 0; k < cp; k++) wp2[(size_t)k * P + p] = m.p2.w[(size_t)p * cp + k];
    a.w_p2 = upload_f(wp2); a.P = P;
    a.v1_off = cp + cg; a.c_v1 = cv;
    a.v1_scale = upload_f(m.v1_bn.scale); a.v1_shift = upload_f(m.v1_bn.bias); a.v1_act = m.v1_act;
    a.w_own = upload_f(m.own.w);
    a.mask = mask_;
    a.out = out; a.row_len = rl; a.own_off = P * (HW + 1) + 3 + S;
    if (m.p1_act != m.v1_act) throw std::runtime_error("policy p1 and value v1 activations differ");
    Op op;
    op.launch = [=](hipStream_t s, int B) { launch_head_spatial(a, B, s); };
    op.cls = "head";
    op.bytes_row = (double)HW * (cp + cv) * 4;
    ops_.push_back(op);
  }

  // Winograd workspace, sized by the largest convolution.
  // Zeroed once: padding tile rows are read by the GEMMs but never written.
  // A workspace plan clears them before every forward instead (its memory is shared and keeps older contents).
  if (wino_v_elems_) {
    wino_v_ = alloc_bytes(wino_v_elems_ * tsize());
    if (primary_) zero_.emplace_back(wino_v_, wino_v_elems_ * tsize());
    else KGX_HIP(hipMemset(wino_v_, 0, wino_v_elems_ * tsize()));
  }
  if (wino_m_elems_) {
    wino_m_ = alloc_f(wino_m_elems_);
    if (primary_) zero_.emplace_back(wino_m_, wino_m_elems_ * 4);
    else KGX_HIP(hipMemset(wino_m_, 0, wino_m_elems_ * 4));
  }
  // Each kernel that can touches the weights of the next op that has weights (at most two ops ahead) into L2.
  if (l2_prefetch_) {
    for (size_t i = 0; i < ops_.size(); i++) {
      if (!ops_[i].pf_sink) continue;
      for (size_t j = i + 1; j < ops_.size() && j <= i + 1; j++) {
        if (!ops_[j].w || ops_[j].w_bytes > (size_t)INT32_MAX) continue;
        ops_[i].pf_sink->pf = (const char*)ops_[j].w;
        ops_[i].pf_sink->pf_bytes = (int)ops_[j].w_bytes;
        break;
      }
    }
  }
  if (!primary_) KGX_HIP(hipDeviceSynchronize());
}

void Net::run_ops(int B, hipStream_t s) {
  if (!profiling_) {
    for (const Op& op : ops_) op.launch(s, B);
    return;
  }
  // Events around every op, plus a pair that the op's kernels record themselves (LaunchTiming, launch_k), whose
  // span then excludes the dispatch latency of an eager launch.
  const size_t need = 4 * ops_.size();
  while (events_.size() < need) {
    hipEvent_t e;
    KGX_HIP(hipEventCreate(&e));
    events_.push_back(e);
  }
  std::vector<char> kernel_timed(ops_.size(), 0);
  for (size_t k = 0; k < ops_.size(); k++) {
    KGX_HIP(hipEventRecord(events_[4 * k], s));
    g_launch_timing = LaunchTiming{events_[4 * k + 2], events_[4 * k + 3], false};
    try {
      ops_[k].launch(s, B);
    } catch (...) {
      g_launch_timing = LaunchTiming{};
      throw;
    }
    kernel_timed[k] = g_launch_timing.used;
    g_launch_timing = LaunchTiming{};
    KGX_HIP(hipEventRecord(events_[4 * k + 1], s));
  }
  KGX_HIP(hipStreamSynchronize(s));
  for (size_t k = 0; k < ops_.size(); k++) {
    float ms = 0.f;
    if (kernel_timed[k]) KGX_HIP(hipEventElapsedTime(&ms, events_[4 * k + 2], events_[4 * k + 3]));
    else KGX_HIP(hipEventElapsedTime(&ms, events_[4 * k], events_[4 * k + 1]));
    ProfileClass& pc = profile_[ops_[k].cls];
    pc.name = ops_[k].cls;
    pc.launches++;
    pc.ms += ms;
    pc.flops += ops_[k].flops_row * B;
    pc.bytes += ops_[k].bytes_row * B + ops_[k].bytes_fixed;
    if (ops_[k].out && ops_[k].out->emit.scale)
      pc.bytes += (double)HW * ops_[k].out_c * tsize() * B * (ops_[k].out->emit.out_lo ? 2 : 1);
  }
}

void Net::forward_eager(int B, hipStream_t s) {
  if (!primary_ || !fits()) throw std::runtime_error("internal: not a runnable workspace plan");
  if (B < 1 || B > max_batch_) throw std::runtime_error("batch size out of range");
  for (const auto& z : zero_) launch_fill_zero(z.first, z.second, s);
  for (const Op& op : ops_) op.launch(s, B);
}

void Net::forward(int B, hipStream_t s) {
  if (B < 1 || B > max_batch_) throw std::runtime_error("batch size out of range");
  KGX_HIP(hipSetDevice(device_));
  if (profiling_ || !use_graphs_) {
    run_ops(B, s);
    return;
  }
  auto it = graphs_.find(B);
  if (it == graphs_.end()) {
    hipGraph_t graph;
    KGX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
      run_ops(B, s);
    } catch (...) {
      hipGraph_t g2;
      (void)hipStreamEndCapture(s, &g2);
      if (g2) (void)hipGraphDestroy(g2);
      throw;
    }
    KGX_HIP(hipStreamEndCapture(s, &graph));
    hipGraphExec_t exec;
    KGX_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    (void)hipGraphDestroy(graph);
    it = graphs_.emplace(B, exec).first;
  }
  KGX_HIP(hipGraphLaunch(it->second, s));
}

}  // namespace kgx
