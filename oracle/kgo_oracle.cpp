// CPU oracle for the KataGo network forward pass.
//
// TEST INFRASTRUCTURE ONLY. Only tests/, the smoke check and the benchmark's CPU-baseline leg load this
// library; the product path (katago-rs_amd/csrc) never includes, links or calls it.
//
// A from-scratch restatement, in plain loops, of the graph that tools/bin2onnx/bin2onnx.py builds
// (GraphBuilder, bin2onnx.py:1088-1531), evaluated in double (kgo_forward_f64, the parity reference) or
// float (kgo_forward_f32, the CPU baseline), on the NCHW layout of the reference. It has its own parser of
// KataGo's model-file format (mirroring bin2onnx.py:60-1069) so that it shares no code with the product.
// Next to the forward pass it restates the reference's Winograd F(4x4,3x3) transforms
// (crates/katago-nn-burn/src/wino/kernels.rs:36-69, 79-179, 312-384), the symmetry copy
// (crates/katago-core/src/neuralnet/nninputs.rs:756-850), the batch-bucket choice
// (crates/katago-nn-burn/src/backend.rs:82-84) and the output unpacking of copy_outputs (backend.rs:622-731).
//
// Pinning (tests/test_oracle.py): the Winograd restatement equals direct convolution in double (closed
// form); the direct convolution, matmuls, softmax attention and RMSNorm equal torch's library routines in
// float64 on the same weights; pooling constants reduce to their closed forms on a full board; symmetry
// is brute-forced against the dihedral group; whole-forward invariants (row independence, identity of a
// residual block with a zero final conv) hold. Parity unpinned against the reference's own numbers: the
// reference's fixtures need network weights that are not available (see DESIGN.md of the repository).

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>
#include <stdexcept>
#include <algorithm>
#include <zlib.h>

namespace {

constexpr int POS = 19;
constexpr int HW = POS * POS;

// ---------------------------------------------------------------------------------------------------------
// Model file reader (bin2onnx.py:60-125: whitespace tokens, floats as "@BIN@" blocks or text tokens)
// ---------------------------------------------------------------------------------------------------------

struct Reader {
  const uint8_t* d;
  size_t n;
  size_t pos = 0;
  bool bin;
  static bool ws(uint8_t c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\v' || c == '\f'; }
  void skip() { while (pos < n && ws(d[pos])) pos++; }
  std::string token() {
    skip();
    size_t s = pos;
    while (pos < n && !ws(d[pos])) pos++;
    if (pos == s) throw std::runtime_error("Unexpected end of model file");
    return std::string((const char*)d + s, pos - s);
  }
  int i() {
    std::string t = token();
    char* e = nullptr;
    long v = strtol(t.c_str(), &e, 10);
    if (*e) throw std::runtime_error("expected integer, got " + t);
    return (int)v;
  }
  float f() {
    std::string t = token();
    return strtof(t.c_str(), nullptr);
  }
  bool b() {
    int v = i();
    if (v != 0 && v != 1) throw std::runtime_error("expected bool");
    return v == 1;
  }
  std::vector<float> floats(size_t cnt, const std::string& name) {
    std::vector<float> out(cnt);
    if (!bin) {
      for (size_t k = 0; k < cnt; k++) out[k] = f();
    } else {
      int before = 0;
      while (true) {
        if (pos >= n) throw std::runtime_error(name + ": could not find binary float block");
        uint8_t c = d[pos++];
        if (c == '@') break;
        if (++before > 100) throw std::runtime_error(name + ": no @BIN@ header");
      }
      if (pos + 4 > n || memcmp(d + pos, "BIN@", 4) != 0) throw std::runtime_error(name + ": bad binary header");
      pos += 4;
      if (pos + 4 * cnt > n) throw std::runtime_error(name + ": truncated float block");
      memcpy(out.data(), d + pos, 4 * cnt);
      pos += 4 * cnt;
    }
    for (float v : out)
      if (!std::isfinite(v)) throw std::runtime_error(name + ": non-finite weight");
    return out;
  }
};

enum ActKind { A_ID = 0, A_RELU = 1, A_MISH = 2, A_SILU = 3 };

struct Conv { int ky = 0, kx = 0, ic = 0, oc = 0, dy = 1, dx = 1; std::vector<float> w; };  // [oc][ic][ky][kx]
struct BN { int c = 0; std::vector<float> ms, mb; };  // merged scale/bias in float (bin2onnx.py:179-184)
struct MatMul { int ic = 0, oc = 0; std::vector<float> w; };  // [ic][oc]
struct MatBias { int c = 0; std::vector<float> b; };

enum BlockKind { B_RES, B_GPOOL, B_NBT, B_ATTN, B_FFN };

struct Block {
  BlockKind kind;
  BN pre_bn; int pre_act = A_ID;
  Conv regular, gconv, final_;  // nbt: regular = pre conv, final_ = post conv
  BN gbn; int gact = A_ID; MatMul gmul;
  BN mid_bn; int mid_act = A_ID;  // nbt: post bn / act
  std::vector<Block> inner;
  // transformer attention
  int heads = 0, kvh = 0, dq = 0, dv = 0; bool rope = false, learnable = false; float theta = 0;
  std::vector<float> freqs;  // [kvh][dq/2][2]
  std::vector<float> ln_w; float ln_eps = 0;
  MatMul q, k, v, o;
  // transformer ffn
  int ffn_c = 0; bool swiglu = false; MatMul l1, lg, l2;
  int in_c = 0;
};

struct Model {
  std::string name;
  int version = 0, nin = 0, nglob = 0, nmeta = 0, meta_ver = 0;
  int trunk_c = 0;
  Conv stem; MatMul stem_mm;
  MatMul m1, m2, m3; MatBias mb1, mb2; int ma1 = A_ID, ma2 = A_ID;
  std::vector<Block> blocks;
  int tip_kind = 0;  // 0 bn, 1 rmsnorm
  BN tip_bn;
  int rms_c = 0; float rms_eps = 0; bool rms_spatial = false; std::vector<float> rms_gamma, rms_beta;
  int tip_act = A_ID;
  int P = 1, S = 1;
  Conv p1, g1, p2; BN g1bn, p1bn; int g1act = A_ID, p1act = A_ID; MatMul gpool_bias, pass1, pass2; MatBias passb; int passact = A_ID;
  Conv v1, own; BN v1bn; int v1act = A_ID; MatMul v2, v3, sv3; MatBias v2b, v3b, sv3b; int v2act = A_ID;
  int row_len() const { return P * (HW + 1) + 3 + S + HW; }
};

void check(bool c, const std::string& msg) { if (!c) throw std::runtime_error(msg); }

Conv parse_conv(Reader& r) {
  std::string name = r.token();
  Conv c;
  c.ky = r.i(); c.kx = r.i(); c.ic = r.i(); c.oc = r.i(); c.dy = r.i(); c.dx = r.i();
  check(c.ky > 0 && c.kx > 0 && c.ky % 2 == 1 && c.kx % 2 == 1, name + ": bad conv size");
  check(c.ic > 0 && c.oc > 0 && c.dy > 0 && c.dx > 0, name + ": bad conv channels/dilation");
  std::vector<float> raw = r.floats((size_t)c.ky * c.kx * c.ic * c.oc, name);
  c.w.resize(raw.size());
  // File order y, x, ic, oc -> [oc][ic][y][x].
  for (int y = 0; y < c.ky; y++)
    for (int x = 0; x < c.kx; x++)
      for (int i = 0; i < c.ic; i++)
        for (int o = 0; o < c.oc; o++)
          c.w[(((size_t)o * c.ic + i) * c.ky + y) * c.kx + x] = raw[(((size_t)y * c.kx + x) * c.ic + i) * c.oc + o];
  return c;
}

BN parse_bn(Reader& r) {
  std::string name = r.token();
  BN b;
  b.c = r.i();
  float eps = r.f();
  bool has_scale = r.b(), has_bias = r.b();
  check(b.c >= 1 && eps > 0, name + ": bad bn");
  auto mean = r.floats(b.c, name), var = r.floats(b.c, name);
  std::vector<float> scale = has_scale ? r.floats(b.c, name) : std::vector<float>(b.c, 1.0f);
  std::vector<float> bias = has_bias ? r.floats(b.c, name) : std::vector<float>(b.c, 0.0f);
  b.ms.resize(b.c); b.mb.resize(b.c);
  for (int i = 0; i < b.c; i++) {
    float s = scale[i] / std::sqrt(var[i] + eps);  // float arithmetic, as computeMerged
    b.ms[i] = s;
    b.mb[i] = bias[i] - s * mean[i];
  }
  return b;
}

int parse_act(Reader& r, int version) {
  r.token();
  if (version < 11) return A_RELU;
  std::string k = r.token();
  if (k == "ACTIVATION_IDENTITY") return A_ID;
  if (k == "ACTIVATION_RELU") return A_RELU;
  if (k == "ACTIVATION_MISH") return A_MISH;
  if (k == "ACTIVATION_SILU") return A_SILU;
  throw std::runtime_error("unknown activation " + k);
}

MatMul parse_mm(Reader& r) {
  std::string name = r.token();
  MatMul m; m.ic = r.i(); m.oc = r.i();
  check(m.ic > 0 && m.oc > 0, name + ": bad matmul");
  m.w = r.floats((size_t)m.ic * m.oc, name);
  return m;
}

MatBias parse_mb(Reader& r) {
  std::string name = r.token();
  MatBias b; b.c = r.i();
  check(b.c > 0, name + ": bad matbias");
  b.b = r.floats(b.c, name);
  return b;
}

void parse_tf_ln(Reader& r, Block& b) {
  std::string name = r.token();
  int c = r.i();
  b.ln_eps = r.f();
  check(c >= 1, name + ": bad rmsnorm");
  b.ln_w = r.floats(c, name);
}

std::vector<Block> parse_stack(Reader& r, int version, int nblocks, int c);

Block parse_block(Reader& r, int version, int c) {
  std::string kind = r.token();
  Block b;
  b.in_c = c;
  if (kind == "ordinary_block") {
    b.kind = B_RES; r.token();
    b.pre_bn = parse_bn(r); b.pre_act = parse_act(r, version);
    b.regular = parse_conv(r);
    b.mid_bn = parse_bn(r); b.mid_act = parse_act(r, version);
    b.final_ = parse_conv(r);
    check(b.regular.ic == c && b.final_.oc == c && b.final_.ic == b.regular.oc, "residual block channels");
  } else if (kind == "gpool_block") {
    b.kind = B_GPOOL; r.token();
    b.pre_bn = parse_bn(r); b.pre_act = parse_act(r, version);
    b.regular = parse_conv(r); b.gconv = parse_conv(r);
    b.gbn = parse_bn(r); b.gact = parse_act(r, version);
    b.gmul = parse_mm(r);
    b.mid_bn = parse_bn(r); b.mid_act = parse_act(r, version);
    b.final_ = parse_conv(r);
    check(b.gmul.ic == 3 * b.gconv.oc && b.gmul.oc == b.regular.oc && b.final_.oc == c, "gpool block channels");
  } else if (kind == "nested_bottleneck_block") {
    b.kind = B_NBT; r.token();
    int nb = r.i();
    check(nb >= 1, "nested bottleneck num blocks");
    b.pre_bn = parse_bn(r); b.pre_act = parse_act(r, version);
    b.regular = parse_conv(r);
    b.inner = parse_stack(r, version, nb, b.regular.oc);
    b.mid_bn = parse_bn(r); b.mid_act = parse_act(r, version);
    b.final_ = parse_conv(r);
    check(b.final_.oc == c && b.regular.ic == c, "nested bottleneck channels");
  } else if (kind == "transformer_attention_block") {
    b.kind = B_ATTN; r.token();
    b.heads = r.i(); b.kvh = r.i(); b.dq = r.i(); b.dv = r.i();
    b.rope = r.i() != 0; b.learnable = r.i() != 0;
    check(b.heads >= 1 && b.kvh >= 1 && b.heads % b.kvh == 0 && b.dq >= 1 && b.dv >= 1, "attention heads");
    check(!b.rope || b.dq % 2 == 0, "odd qHeadDim with RoPE");
    parse_tf_ln(r, b);
    b.q = parse_mm(r); b.k = parse_mm(r); b.v = parse_mm(r); b.o = parse_mm(r);
    check(b.q.oc == b.heads * b.dq && b.k.oc == b.kvh * b.dq && b.v.oc == b.kvh * b.dv && b.o.ic == b.heads * b.dv, "attention projections");
    if (b.rope) {
      r.token();
      if (b.learnable) {
        int a = r.i(), p = r.i(), two = r.i();
        check(a == b.kvh && p == b.dq / 2 && two == 2, "rope freqs shape");
        b.freqs = r.floats((size_t)a * p * 2, "ropefreqs");
      } else {
        b.theta = r.f();
        check(b.theta > 0, "rope theta");
      }
    }
  } else if (kind == "transformer_ffn_block") {
    b.kind = B_FFN; r.token();
    int cc = r.i(); b.ffn_c = r.i(); b.swiglu = r.i() != 0;
    check(cc == c, "ffn channels");
    parse_tf_ln(r, b);
    b.l1 = parse_mm(r);
    if (b.swiglu) b.lg = parse_mm(r);
    b.l2 = parse_mm(r);
  } else {
    throw std::runtime_error("unknown block kind " + kind);
  }
  return b;
}

std::vector<Block> parse_stack(Reader& r, int version, int nblocks, int c) {
  std::vector<Block> out;
  for (int i = 0; i < nblocks; i++) out.push_back(parse_block(r, version, c));
  return out;
}

Model parse_model(Reader& r) {
  Model m;
  m.name = r.token();
  m.version = r.i();
  check(m.version >= 3 && m.version <= 17, "unsupported model version");
  m.nin = r.i(); m.nglob = r.i();
  if (m.version >= 13)
    for (int k = 0; k < 7; k++) r.f();
  if (m.version >= 15) {
    m.meta_ver = r.i();
    check(m.meta_ver == 0 || m.meta_ver == 1, "meta encoder version");
    m.nmeta = m.meta_ver ? 192 : 0;
    for (int k = 0; k < 7; k++) r.i();
  }
  // Trunk.
  r.token();
  int nblocks = r.i();
  m.trunk_c = r.i();
  r.i(); r.i(); r.i(); r.i();
  if (m.version >= 15) {
    m.tip_kind = r.i();
    for (int k = 0; k < 5; k++) check(r.i() == 0, "trunk option");
  }
  m.stem = parse_conv(r);
  m.stem_mm = parse_mm(r);
  if (m.meta_ver > 0) {
    r.token();
    check(r.i() == 192, "meta channels");
    m.m1 = parse_mm(r); m.mb1 = parse_mb(r); m.ma1 = parse_act(r, m.version);
    m.m2 = parse_mm(r); m.mb2 = parse_mb(r); m.ma2 = parse_act(r, m.version);
    m.m3 = parse_mm(r);
  }
  m.blocks = parse_stack(r, m.version, nblocks, m.trunk_c);
  if (m.tip_kind == 0) {
    m.tip_bn = parse_bn(r);
  } else {
    r.token();
    m.rms_c = r.i(); m.rms_eps = r.f(); m.rms_spatial = r.i() != 0;
    check(r.i() == 0, "grouped rmsnorm");
    m.rms_gamma = r.floats(m.rms_c, "rms"); m.rms_beta = r.floats(m.rms_c, "rms");
  }
  m.tip_act = parse_act(r, m.version);
  // Policy head.
  r.token();
  if (m.version >= 17) {
    m.P = r.i();
    for (int k = 0; k < 3; k++) r.i();
  } else if (m.version == 16) m.P = 4;
  else if (m.version >= 12) m.P = 2;
  else m.P = 1;
  m.p1 = parse_conv(r); m.g1 = parse_conv(r);
  m.g1bn = parse_bn(r); m.g1act = parse_act(r, m.version);
  m.gpool_bias = parse_mm(r);
  m.p1bn = parse_bn(r); m.p1act = parse_act(r, m.version);
  m.p2 = parse_conv(r);
  m.pass1 = parse_mm(r);
  if (m.version >= 15) {
    m.passb = parse_mb(r); m.passact = parse_act(r, m.version); m.pass2 = parse_mm(r);
  }
  // Value head.
  r.token();
  if (m.version >= 17)
    for (int k = 0; k < 3; k++) r.i();
  m.v1 = parse_conv(r); m.v1bn = parse_bn(r); m.v1act = parse_act(r, m.version);
  m.v2 = parse_mm(r); m.v2b = parse_mb(r); m.v2act = parse_act(r, m.version);
  m.v3 = parse_mm(r); m.v3b = parse_mb(r);
  m.sv3 = parse_mm(r); m.sv3b = parse_mb(r);
  m.own = parse_conv(r);
  m.S = m.sv3.oc;
  r.skip();
  check(r.pos == r.n, "trailing bytes in model file");
  return m;
}

// ---------------------------------------------------------------------------------------------------------
// Forward pass (NCHW, Real = double or float)
// ---------------------------------------------------------------------------------------------------------

template <typename R>
R act(R a, int kind) {
  switch (kind) {
    case A_RELU: return a > R(0) ? a : R(0);
    case A_MISH: {
      R sp = a > R(20) ? a : std::log1p(std::exp(a));  // softplus with burn's threshold
      return a * std::tanh(sp);
    }
    case A_SILU: return a / (std::exp(-a) + R(1));      // bin2onnx.py:1163-1168
    default: return a;
  }
}

// Rounding of a value to a 16-bit floating-point operand, round-to-nearest-even: float16 (11 significant bits,
// normal range from 2^-14, subnormal quantum 2^-24, overflow above 65504 to infinity) or bfloat16 (8 significant
// bits, float32's exponent range). Used to emulate a forward pass whose GEMM operands are 16-bit.
enum { Q_NONE = 0, Q_F16 = 1, Q_BF16 = 2 };
// Layer classes of the rounding points: the stem convolution, the 3x3 convolutions of residual and gpool
// blocks, a gpool block's pooling convolution, a nested bottleneck's entry and exit 1x1 convolutions, and
// the transformer token GEMMs with the attention operands.
enum { QC_STEM = 1, QC_CONV3 = 2, QC_GCONV = 4, QC_NBT_IN = 8, QC_NBT_OUT = 16, QC_TOKEN = 32, QC_ALL = 63 };
double round_operand(double x, int q) {
  if (q == Q_NONE || x == 0.0 || !std::isfinite(x)) return x;
  int e;
  std::frexp(x, &e);  // |x| = f 2^e, f in [0.5, 1)
  const int bits = q == Q_F16 ? 11 : 8;
  int qe = e - bits;
  if (q == Q_F16) qe = std::max(qe, -24);
  const double r = std::nearbyint(std::ldexp(x, -qe)) * std::ldexp(1.0, qe);  // default rounding: to even
  if (q == Q_F16 && std::fabs(r) > 65504.0) return std::copysign(INFINITY, x);
  return r;
}

template <typename R>
struct Fwd {
  const Model& m;
  int n;
  std::vector<R> mask, area, s1, s2;  // mask [n][HW]
  int threads;
  // Operand emulation (double only): the trunk's convolution and token-GEMM operands (inputs and weights), the
  // q/k/v projections and the attention output are rounded to 16 bits; accumulation, residual streams, pooling,
  // normalization statistics and the heads stay exact. qa / qw choose the rounding of activations / weights.
  // qclass restricts the rounding to the layer classes whose QC_* bit it holds (all by default), which
  // attributes a 16-bit forward pass's error to its rounding points.
  int qa = Q_NONE, qw = Q_NONE;
  int qclass = QC_ALL, qclass_w = QC_ALL;  // activation and weight rounding classes

  Fwd(const Model& mm, int nn, int th) : m(mm), n(nn), threads(th) {}

  R ra(R v) const { return qa ? (R)round_operand((double)v, qa) : v; }
  R rw(R v) const { return qw ? (R)round_operand((double)v, qw) : v; }
  bool tokq() const { return (qclass & QC_TOKEN) != 0; }
  bool tokq_w() const { return (qclass_w & QC_TOKEN) != 0; }

  // "same" convolution, zero padding, on [n][C][HW]; `cls` is the QC_* class of a trunk convolution (16-bit
  // operands when emulated), 0 for the float convolutions of the heads.
  std::vector<R> conv(const std::vector<R>& x0, const Conv& c, int cls = 0) {
    const bool half = cls != 0 && (qclass & cls) != 0;
    std::vector<R> xr;
    if (half && qa) {
      xr = x0;
      for (auto& v : xr) v = ra(v);
    }
    const std::vector<R>& x = (half && qa) ? xr : x0;
    const bool hw = cls != 0 && (qclass_w & cls) != 0 && qw;
    std::vector<R> out((size_t)n * c.oc * HW, R(0));
    const int py = (c.ky / 2) * c.dy, px = (c.kx / 2) * c.dx;
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
    for (int b = 0; b < n; b++)
      for (int o = 0; o < c.oc; o++) {
        R* acc = &out[((size_t)b * c.oc + o) * HW];
        for (int i = 0; i < c.ic; i++) {
          const R* in = &x[((size_t)b * c.ic + i) * HW];
          for (int ky = 0; ky < c.ky; ky++) {
            const int oy = ky * c.dy - py;
            for (int kx = 0; kx < c.kx; kx++) {
              const int ox = kx * c.dx - px;
              R w = (R)c.w[(((size_t)o * c.ic + i) * c.ky + ky) * c.kx + kx];
              if (hw) w = rw(w);
              const int y0 = std::max(0, -oy), y1 = std::min(POS, POS - oy);
              const int x0 = std::max(0, -ox), x1 = std::min(POS, POS - ox);
              for (int y = y0; y < y1; y++) {
                R* arow = acc + y * POS;
                const R* irow = in + (y + oy) * POS + ox;
                for (int xx = x0; xx < x1; xx++) arow[xx] += w * irow[xx];
              }
            }
          }
        }
      }
    return out;
  }

  std::vector<R> bn_act_mask(const std::vector<R>& x, const BN& bn, int a) {
    std::vector<R> out(x.size());
    for (int b = 0; b < n; b++)
      for (int c = 0; c < bn.c; c++) {
        const R s = bn.ms[c], bb = bn.mb[c];
        for (int p = 0; p < HW; p++) {
          size_t idx = ((size_t)b * bn.c + c) * HW + p;
          out[idx] = act<R>(x[idx] * s + bb, a) * mask[(size_t)b * HW + p];
        }
      }
    return out;
  }

  // [n][ic] x [ic][oc] -> [n][oc]
  std::vector<R> matmul(const std::vector<R>& x, const MatMul& mm) {
    std::vector<R> out((size_t)n * mm.oc, R(0));
    for (int b = 0; b < n; b++)
      for (int i = 0; i < mm.ic; i++) {
        const R xv = x[(size_t)b * mm.ic + i];
        for (int o = 0; o < mm.oc; o++) out[(size_t)b * mm.oc + o] += xv * (R)mm.w[(size_t)i * mm.oc + o];
      }
    return out;
  }

  void matbias(std::vector<R>& x, const MatBias& mb) {
    for (int b = 0; b < n; b++)
      for (int c = 0; c < mb.c; c++) x[(size_t)b * mb.c + c] += (R)mb.b[c];
  }

  void act_inplace(std::vector<R>& x, int a) {
    for (auto& v : x) v = act<R>(v, a);
  }

  // gpool (bin2onnx.py:1230-1238): [mean, mean * s1, max(x + mask*1e4 - 1e4)] -> [n][3C]
  std::vector<R> gpool(const std::vector<R>& x, int C) {
    std::vector<R> out((size_t)n * 3 * C);
    for (int b = 0; b < n; b++)
      for (int c = 0; c < C; c++) {
        R sum = 0, mx = -INFINITY;
        for (int p = 0; p < HW; p++) {
          R v = x[((size_t)b * C + c) * HW + p];
          sum += v;
          R bias = mask[(size_t)b * HW + p] * R(1e4) - R(1e4);
          mx = std::max(mx, v + bias);
        }
        R mean = sum / area[b];
        out[(size_t)b * 3 * C + c] = mean;
        out[(size_t)b * 3 * C + C + c] = mean * s1[b];
        out[(size_t)b * 3 * C + 2 * C + c] = mx;
      }
    return out;
  }

  // value pool (bin2onnx.py:1240-1247): [mean, mean * s1, mean * s2]
  std::vector<R> value_pool(const std::vector<R>& x, int C) {
    std::vector<R> out((size_t)n * 3 * C);
    for (int b = 0; b < n; b++)
      for (int c = 0; c < C; c++) {
        R sum = 0;
        for (int p = 0; p < HW; p++) sum += x[((size_t)b * C + c) * HW + p];
        R mean = sum / area[b];
        out[(size_t)b * 3 * C + c] = mean;
        out[(size_t)b * 3 * C + C + c] = mean * s1[b];
        out[(size_t)b * 3 * C + 2 * C + c] = mean * s2[b];
      }
    return out;
  }

  void add_nc_bias(std::vector<R>& x, const std::vector<R>& bias, int C) {
    for (int b = 0; b < n; b++)
      for (int c = 0; c < C; c++)
        for (int p = 0; p < HW; p++) x[((size_t)b * C + c) * HW + p] += bias[(size_t)b * C + c];
  }

  void add(std::vector<R>& x, const std::vector<R>& y) {
    for (size_t k = 0; k < x.size(); k++) x[k] += y[k];
  }

  // --- transformer blocks on tokens [n][HW][C] ---

  std::vector<R> to_tokens(const std::vector<R>& x, int C) {
    std::vector<R> t(x.size());
    for (int b = 0; b < n; b++)
      for (int c = 0; c < C; c++)
        for (int p = 0; p < HW; p++) t[((size_t)b * HW + p) * C + c] = x[((size_t)b * C + c) * HW + p];
    return t;
  }
  std::vector<R> to_nchw(const std::vector<R>& t, int C) {
    std::vector<R> x(t.size());
    for (int b = 0; b < n; b++)
      for (int c = 0; c < C; c++)
        for (int p = 0; p < HW; p++) x[((size_t)b * C + c) * HW + p] = t[((size_t)b * HW + p) * C + c];
    return x;
  }

  // rows [n*HW][ic] x [ic][oc] (operands rounded when emulated)
  std::vector<R> tok_matmul(const std::vector<R>& t, const MatMul& mm) {
    const size_t rows = (size_t)n * HW;
    std::vector<R> out(rows * mm.oc, R(0));
    std::vector<R> wr((size_t)mm.ic * mm.oc);
    const bool q = tokq(), qwt = tokq_w();
    for (size_t k = 0; k < wr.size(); k++) wr[k] = qwt ? rw((R)mm.w[k]) : (R)mm.w[k];
#pragma omp parallel for schedule(static) num_threads(threads)
    for (long r = 0; r < (long)rows; r++) {
      R* o = &out[r * mm.oc];
      for (int i = 0; i < mm.ic; i++) {
        const R xv = q ? ra(t[r * mm.ic + i]) : t[r * mm.ic + i];
        const R* w = &wr[(size_t)i * mm.oc];
        for (int j = 0; j < mm.oc; j++) o[j] += xv * w[j];
      }
    }
    return out;
  }

  // TransformerRMSNormLayer (bin2onnx.py:1338-1348)
  std::vector<R> tf_rmsnorm(const std::vector<R>& t, const Block& bl, int C) {
    std::vector<R> out(t.size());
    for (size_t r = 0; r < (size_t)n * HW; r++) {
      R ss = 0;
      for (int c = 0; c < C; c++) ss += t[r * C + c] * t[r * C + c];
      R rms = R(1) / std::sqrt(ss / R(C) + R(bl.ln_eps));
      R mk = mask[r];
      for (int c = 0; c < C; c++) out[r * C + c] = t[r * C + c] * rms * (R)bl.ln_w[c] * mk;
    }
    return out;
  }

  // RoPE tables (bin2onnx.py:449-485), float like the reference: [tables][pairs][HW]
  void rope_tables(const Block& bl, std::vector<float>& cs, std::vector<float>& sn, int& ntab) {
    const int pairs = bl.dq / 2;
    if (bl.learnable) {
      ntab = bl.kvh;
      cs.assign((size_t)ntab * pairs * HW, 0.f); sn = cs;
      for (int h = 0; h < bl.kvh; h++)
        for (int p = 0; p < pairs; p++) {
          const float fx = bl.freqs[((size_t)h * pairs + p) * 2], fy = bl.freqs[((size_t)h * pairs + p) * 2 + 1];
          for (int y = 0; y < POS; y++)
            for (int x = 0; x < POS; x++) {
              float ang = (float)x * fx + (float)y * fy;
              cs[((size_t)h * pairs + p) * HW + y * POS + x] = (float)std::cos((double)ang);
              sn[((size_t)h * pairs + p) * HW + y * POS + x] = (float)std::sin((double)ang);
            }
        }
    } else {
      ntab = 1;
      cs.assign((size_t)pairs * HW, 0.f); sn = cs;
      const int per_dim = pairs / 2;
      const float dim_half = (float)(bl.dq / 2);
      for (int p = 0; p < pairs; p++) {
        const int padj = p < per_dim ? p : p - per_dim;
        const float expo = (float)(2 * padj) / dim_half;
        const float powv = (float)std::pow((double)bl.theta, (double)expo);
        const float freq = 1.0f / powv;
        for (int y = 0; y < POS; y++)
          for (int x = 0; x < POS; x++) {
            const float pos = p < per_dim ? (float)y : (float)x;
            const float ang = pos * freq;
            cs[(size_t)p * HW + y * POS + x] = (float)std::cos((double)ang);
            sn[(size_t)p * HW + y * POS + x] = (float)std::sin((double)ang);
          }
      }
    }
  }

  // TransformerAttentionBlock (bin2onnx.py:1357-1421), RoPE on interleaved pairs (2p, 2p+1).
  void attention_block(std::vector<R>& t, const Block& bl, int C) {
    std::vector<R> xn = tf_rmsnorm(t, bl, C);
    std::vector<R> q = tok_matmul(xn, bl.q), k = tok_matmul(xn, bl.k), v = tok_matmul(xn, bl.v);
    // With 16-bit storage: v is stored as projected; q and k are stored once, after rotation and scaling below.
    const bool q16 = qa && tokq();
    if (q16)
      for (auto& z : v) z = ra(z);
    const int H = bl.heads, KV = bl.kvh, dq = bl.dq, dv = bl.dv, g = H / KV;
    if (bl.rope) {
      std::vector<float> cs, sn; int ntab;
      rope_tables(bl, cs, sn, ntab);
      const int pairs = dq / 2;
      auto rot = [&](std::vector<R>& z, int nheads, bool is_q) {
        for (int b = 0; b < n; b++)
          for (int s = 0; s < HW; s++)
            for (int h = 0; h < nheads; h++) {
              int tab = 0;
              if (bl.learnable) tab = is_q ? h * KV / H : h;
              R* zz = &z[((size_t)b * HW + s) * nheads * dq + (size_t)h * dq];
              for (int p = 0; p < pairs; p++) {
                R c = cs[((size_t)tab * pairs + p) * HW + s], si = sn[((size_t)tab * pairs + p) * HW + s];
                R x0 = zz[2 * p], x1 = zz[2 * p + 1];
                zz[2 * p] = x0 * c - x1 * si;
                zz[2 * p + 1] = x0 * si + x1 * c;
              }
            }
      };
      rot(q, H, true);
      rot(k, KV, false);
    }
    R scale = (R)(1.0f / std::sqrt((float)dq));
    if (q16) {
      // 16-bit storage feeds the matrix cores: the scaled, rotated queries and the rotated keys are operands.
      for (auto& z : q) z = ra(z * scale);
      for (auto& z : k) z = ra(z);
      scale = R(1);
    }
    std::vector<R> o((size_t)n * HW * H * dv, R(0));
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
    for (int b = 0; b < n; b++)
      for (int h = 0; h < H; h++) {
        const int kh = h / g;
        std::vector<R> sc(HW);
        for (int i = 0; i < HW; i++) {
          const R* qi = &q[((size_t)b * HW + i) * H * dq + (size_t)h * dq];
          R mx = -INFINITY;
          for (int j = 0; j < HW; j++) {
            const R* kj = &k[((size_t)b * HW + j) * KV * dq + (size_t)kh * dq];
            R s = 0;
            for (int d = 0; d < dq; d++) s += qi[d] * kj[d];
            s = s * scale + (mask[(size_t)b * HW + j] * R(3e4) - R(3e4));
            sc[j] = s;
            mx = std::max(mx, s);
          }
          R den = 0;
          for (int j = 0; j < HW; j++) { sc[j] = std::exp(sc[j] - mx); den += sc[j]; }
          R* oi = &o[((size_t)b * HW + i) * H * dv + (size_t)h * dv];
          // With 16-bit storage the unnormalized probabilities are operands too; the denominator stays exact.
          const R inv = R(1) / den;
          for (int j = 0; j < HW; j++) {
            const R pj = (q16 ? ra(sc[j]) : sc[j]) * inv;
            const R* vj = &v[((size_t)b * HW + j) * KV * dv + (size_t)kh * dv];
            for (int d = 0; d < dv; d++) oi[d] += pj * vj[d];
          }
        }
      }
    std::vector<R> out = tok_matmul(o, bl.o);
    for (size_t r = 0; r < (size_t)n * HW; r++)
      for (int c = 0; c < C; c++) t[r * C + c] += out[r * C + c] * mask[r];
  }

  // TransformerFFNBlock (bin2onnx.py:1423-1438). The plain (non-SwiGLU) FFN, which the reference rejects,
  // runs as linear1 -> mish -> linear2.
  void ffn_block(std::vector<R>& t, const Block& bl, int C) {
    std::vector<R> xn = tf_rmsnorm(t, bl, C);
    std::vector<R> a = tok_matmul(xn, bl.l1);
    if (bl.swiglu) {
      std::vector<R> gt = tok_matmul(xn, bl.lg);
      for (size_t k = 0; k < a.size(); k++) a[k] = act<R>(a[k], A_SILU) * gt[k];
    } else {
      for (auto& z : a) z = act<R>(z, A_MISH);
    }
    std::vector<R> out = tok_matmul(a, bl.l2);
    for (size_t r = 0; r < (size_t)n * HW; r++)
      for (int c = 0; c < C; c++) t[r * C + c] += out[r * C + c] * mask[r];
  }

  // --- conv blocks on NCHW [n][C][HW] ---

  void block_stack(std::vector<R>& x, const std::vector<Block>& blocks, int C) {
    size_t i = 0;
    while (i < blocks.size()) {
      if (blocks[i].kind == B_ATTN || blocks[i].kind == B_FFN) {
        std::vector<R> t = to_tokens(x, C);
        while (i < blocks.size() && (blocks[i].kind == B_ATTN || blocks[i].kind == B_FFN)) {
          if (blocks[i].kind == B_ATTN) attention_block(t, blocks[i], C);
          else ffn_block(t, blocks[i], C);
          i++;
        }
        x = to_nchw(t, C);
        continue;
      }
      const Block& bl = blocks[i];
      if (bl.kind == B_RES) {
        std::vector<R> t = bn_act_mask(x, bl.pre_bn, bl.pre_act);
        t = conv(t, bl.regular, QC_CONV3);
        t = bn_act_mask(t, bl.mid_bn, bl.mid_act);
        t = conv(t, bl.final_, QC_CONV3);
        add(x, t);
      } else if (bl.kind == B_GPOOL) {
        std::vector<R> t = bn_act_mask(x, bl.pre_bn, bl.pre_act);
        std::vector<R> reg = conv(t, bl.regular, QC_CONV3);
        std::vector<R> gg = conv(t, bl.gconv, QC_GCONV);
        gg = bn_act_mask(gg, bl.gbn, bl.gact);
        std::vector<R> pooled = gpool(gg, bl.gconv.oc);
        std::vector<R> bias = matmul(pooled, bl.gmul);
        add_nc_bias(reg, bias, bl.regular.oc);
        reg = bn_act_mask(reg, bl.mid_bn, bl.mid_act);
        reg = conv(reg, bl.final_, QC_CONV3);
        add(x, reg);
      } else if (bl.kind == B_NBT) {
        std::vector<R> t = bn_act_mask(x, bl.pre_bn, bl.pre_act);
        t = conv(t, bl.regular, QC_NBT_IN);
        block_stack(t, bl.inner, bl.regular.oc);
        t = bn_act_mask(t, bl.mid_bn, bl.mid_act);
        t = conv(t, bl.final_, QC_NBT_OUT);
        add(x, t);
      }
      i++;
    }
  }

  void run(const float* bin, const float* glob, const float* meta, R* out) {
    const int C = m.trunk_c;
    mask.assign((size_t)n * HW, 0); area.assign(n, 0); s1.assign(n, 0); s2.assign(n, 0);
    for (int b = 0; b < n; b++) {
      R s = 0;
      for (int p = 0; p < HW; p++) {
        mask[(size_t)b * HW + p] = bin[((size_t)b * m.nin) * HW + p];
        s += mask[(size_t)b * HW + p];
      }
      area[b] = s;
      R c = std::sqrt(s) - R(14);
      s1[b] = c * R(0.1);
      s2[b] = c * c * R(0.01) - R(0.1);
    }
    std::vector<R> x((size_t)n * m.nin * HW);
    for (size_t k = 0; k < x.size(); k++) x[k] = bin[k];
    // The device runs 1x1 and 3x3 stems on 16-bit operands and other stems (old nets' 5x5) on float ones.
    const bool stem16 = m.stem.ky == m.stem.kx && (m.stem.ky == 1 || m.stem.ky == 3) && m.stem.dy == 1 && m.stem.dx == 1;
    x = conv(x, m.stem, stem16 ? QC_STEM : 0);
    std::vector<R> g((size_t)n * m.nglob);
    for (size_t k = 0; k < g.size(); k++) g[k] = glob[k];
    add_nc_bias(x, matmul(g, m.stem_mm), C);
    if (m.meta_ver > 0) {
      std::vector<R> mt((size_t)n * 192);
      for (size_t k = 0; k < mt.size(); k++) mt[k] = meta[k];
      mt = matmul(mt, m.m1); matbias(mt, m.mb1); act_inplace(mt, m.ma1);
      mt = matmul(mt, m.m2); matbias(mt, m.mb2); act_inplace(mt, m.ma2);
      mt = matmul(mt, m.m3);
      add_nc_bias(x, mt, C);
    }
    block_stack(x, m.blocks, C);
    // Trunk tip.
    std::vector<R> tip;
    if (m.tip_kind == 0) {
      tip = bn_act_mask(x, m.tip_bn, m.tip_act);
    } else {
      tip.resize(x.size());
      for (int b = 0; b < n; b++) {
        std::vector<R> rms(HW);
        if (!m.rms_spatial) {
          for (int p = 0; p < HW; p++) {
            R ss = 0;
            for (int c = 0; c < C; c++) { R v = x[((size_t)b * C + c) * HW + p]; ss += v * v; }
            rms[p] = R(1) / std::sqrt(ss / R(C) + R(m.rms_eps));
          }
        } else {
          R ss = 0;
          for (int c = 0; c < C; c++)
            for (int p = 0; p < HW; p++) { R v = x[((size_t)b * C + c) * HW + p]; ss += v * v * mask[(size_t)b * HW + p]; }
          R r = R(1) / std::sqrt(ss / (area[b] * R(C)) + R(m.rms_eps));
          for (int p = 0; p < HW; p++) rms[p] = r;
        }
        for (int c = 0; c < C; c++)
          for (int p = 0; p < HW; p++) {
            size_t idx = ((size_t)b * C + c) * HW + p;
            R y = x[idx] * rms[p] * (R)m.rms_gamma[c] + (R)m.rms_beta[c];
            tip[idx] = act<R>(y, m.tip_act) * mask[(size_t)b * HW + p];
          }
      }
    }
    // Policy head (bin2onnx.py:1495-1516).
    std::vector<R> p1 = conv(tip, m.p1);
    std::vector<R> g1 = conv(tip, m.g1);
    g1 = bn_act_mask(g1, m.g1bn, m.g1act);
    std::vector<R> g1p = gpool(g1, m.g1.oc);
    add_nc_bias(p1, matmul(g1p, m.gpool_bias), m.p1.oc);
    p1 = bn_act_mask(p1, m.p1bn, m.p1act);
    std::vector<R> p2 = conv(p1, m.p2);
    std::vector<R> pas;
    if (m.version >= 15) {
      pas = matmul(g1p, m.pass1); matbias(pas, m.passb); act_inplace(pas, m.passact);
      pas = matmul(pas, m.pass2);
    } else {
      pas = matmul(g1p, m.pass1);
    }
    // Value head (bin2onnx.py:1518-1531).
    std::vector<R> v1 = conv(tip, m.v1);
    v1 = bn_act_mask(v1, m.v1bn, m.v1act);
    std::vector<R> vp = value_pool(v1, m.v1.oc);
    std::vector<R> v2 = matmul(vp, m.v2); matbias(v2, m.v2b); act_inplace(v2, m.v2act);
    std::vector<R> val = matmul(v2, m.v3); matbias(val, m.v3b);
    std::vector<R> sc = matmul(v2, m.sv3); matbias(sc, m.sv3b);
    std::vector<R> own = conv(v1, m.own);
    // Rows in the readback order of backend.rs:588-597.
    const int rl = m.row_len();
    for (int b = 0; b < n; b++) {
      R* row = out + (size_t)b * rl;
      for (int p = 0; p < m.P; p++) {
        for (int k = 0; k < HW; k++) row[p * (HW + 1) + k] = p2[((size_t)b * m.P + p) * HW + k];
        row[p * (HW + 1) + HW] = pas[(size_t)b * m.P + p];
      }
      R* r2 = row + m.P * (HW + 1);
      for (int k = 0; k < 3; k++) r2[k] = val[(size_t)b * 3 + k];
      for (int k = 0; k < m.S; k++) r2[3 + k] = sc[(size_t)b * m.S + k];
      for (int k = 0; k < HW; k++) r2[3 + m.S + k] = own[(size_t)b * HW + k];
    }
  }
};

thread_local std::string g_err;

bool inflate_if_gzip(const uint8_t* d, size_t n, std::vector<uint8_t>& out) {
  if (n < 2 || d[0] != 0x1f || d[1] != 0x8b) return false;
  z_stream zs;
  memset(&zs, 0, sizeof(zs));
  if (inflateInit2(&zs, 15 + 32) != Z_OK) throw std::runtime_error("zlib init failed");
  zs.next_in = const_cast<uint8_t*>(d);
  zs.avail_in = (uInt)n;
  out.clear();
  uint8_t buf[1 << 16];
  int rc;
  do {
    zs.next_out = buf;
    zs.avail_out = sizeof(buf);
    rc = inflate(&zs, Z_NO_FLUSH);
    if (rc != Z_OK && rc != Z_STREAM_END) { inflateEnd(&zs); throw std::runtime_error("gzip inflate failed"); }
    out.insert(out.end(), buf, buf + (sizeof(buf) - zs.avail_out));
  } while (rc != Z_STREAM_END);
  inflateEnd(&zs);
  return true;
}

bool contains_bin_marker(const uint8_t* d, size_t n) {
  for (size_t k = 0; k + 5 <= n; k++)
    if (d[k] == '@' && memcmp(d + k, "@BIN@", 5) == 0) return true;
  return false;
}

// Winograd F(4x4,3x3) matrices of the reference, written out from wino/kernels.rs.
// Filter transform rows (kernels.rs:39-48): 1/4 z0, -(z0+z1+z2)/6, (-z0+z1-z2)/6, (z0+2z1+4z2)/24,
// (z0-2z1+4z2)/24, z2.
void wino_g(const double z[3], double o[6]) {
  o[0] = 0.25 * z[0];
  o[1] = (-z[0] - z[1] - z[2]) / 6.0;
  o[2] = (-z[0] + z[1] - z[2]) / 6.0;
  o[3] = (z[0] + 2.0 * z[1] + 4.0 * z[2]) / 24.0;
  o[4] = (z[0] - 2.0 * z[1] + 4.0 * z[2]) / 24.0;
  o[5] = z[2];
}
// Input transform B^T (kernels.rs:151-156).
void wino_bt(const double z[6], double o[6]) {
  o[0] = 4.0 * z[0] - 5.0 * z[2] + z[4];
  o[1] = -4.0 * z[1] - 4.0 * z[2] + z[3] + z[4];
  o[2] = 4.0 * z[1] - 4.0 * z[2] - z[3] + z[4];
  o[3] = -2.0 * z[1] - z[2] + 2.0 * z[3] + z[4];
  o[4] = 2.0 * z[1] - z[2] - 2.0 * z[3] + z[4];
  o[5] = 4.0 * z[1] - 5.0 * z[3] + z[5];
}
// Output transform A^T (kernels.rs:352-355).
void wino_at(const double z[6], double o[4]) {
  o[0] = z[0] + z[1] + z[2] + z[3] + z[4];
  o[1] = (z[1] - z[2]) + 2.0 * (z[3] - z[4]);
  o[2] = (z[1] + z[2]) + 4.0 * (z[3] + z[4]);
  o[3] = (z[1] - z[2]) + 8.0 * (z[3] - z[4]) + z[5];
}

}  // namespace

extern "C" {

const char* kgo_last_error(void) { return g_err.c_str(); }

// Parses a KataGo model file (binary or text floats, optionally gzip-compressed).
int kgo_model_parse(const void* bytes, size_t len, void** out) {
  try {
    std::vector<uint8_t> inflated;
    const uint8_t* d = (const uint8_t*)bytes;
    if (inflate_if_gzip(d, len, inflated)) { d = inflated.data(); len = inflated.size(); }
    Reader r{d, len, 0, contains_bin_marker(d, len)};
    *out = new Model(parse_model(r));
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

void kgo_model_free(void* m) { delete (Model*)m; }

// info: [version, num_input_channels, num_global, num_meta, P, S, row_len, trunk_c]
void kgo_model_info(const void* mp, int* info) {
  const Model& m = *(const Model*)mp;
  info[0] = m.version; info[1] = m.nin; info[2] = m.nglob; info[3] = m.nmeta;
  info[4] = m.P; info[5] = m.S; info[6] = m.row_len(); info[7] = m.trunk_c;
}

// Raw outputs, rows of row_len values (policy P x 362 with pass last, value 3, score S, ownership 361).
int kgo_forward_f64(const void* mp, int n, const float* bin, const float* glob, const float* meta, double* out, int threads) {
  try {
    Fwd<double> f(*(const Model*)mp, n, threads < 1 ? 1 : threads);
    f.run(bin, glob, meta, out);
    return 0;
  } catch (const std::exception& e) { g_err = e.what(); return 1; }
}

// kgo_forward_f64 with 16-bit operand emulation: act_q / weight_q = 0 (exact), 1 (float16), 2 (bfloat16);
// classes / wclasses: the QC_* bits of the layer classes whose activations / weights are rounded.
int kgo_forward_f64_q(const void* mp, int n, const float* bin, const float* glob, const float* meta, double* out,
                      int threads, int act_q, int weight_q, int classes, int wclasses) {
  try {
    Fwd<double> f(*(const Model*)mp, n, threads < 1 ? 1 : threads);
    f.qa = act_q;
    f.qw = weight_q;
    f.qclass = classes;
    f.qclass_w = wclasses;
    f.run(bin, glob, meta, out);
    return 0;
  } catch (const std::exception& e) { g_err = e.what(); return 1; }
}

// kgo_forward_f32 with 16-bit operand emulation (float accumulation, as the device accumulates).
int kgo_forward_f32_q(const void* mp, int n, const float* bin, const float* glob, const float* meta, float* out,
                      int threads, int act_q, int weight_q, int classes, int wclasses) {
  try {
    Fwd<float> f(*(const Model*)mp, n, threads < 1 ? 1 : threads);
    f.qa = act_q;
    f.qw = weight_q;
    f.qclass = classes;
    f.qclass_w = wclasses;
    f.run(bin, glob, meta, out);
    return 0;
  } catch (const std::exception& e) { g_err = e.what(); return 1; }
}

// Rounds values to 16-bit operands in place (q as above).
void kgo_round_operands(double* v, long n, int q) {
  for (long k = 0; k < n; k++) v[k] = round_operand(v[k], q);
}

int kgo_forward_f32(const void* mp, int n, const float* bin, const float* glob, const float* meta, float* out, int threads) {
  try {
    Fwd<float> f(*(const Model*)mp, n, threads < 1 ? 1 : threads);
    f.run(bin, glob, meta, out);
    return 0;
  } catch (const std::exception& e) { g_err = e.what(); return 1; }
}

// Direct "same" convolution in double: x [n][ic][19][19], w [oc][ic][k][k] -> y [n][oc][19][19].
void kgo_conv_direct_f64(int n, int ic, int oc, int k, const double* x, const double* w, double* y) {
  const int pad = k / 2;
  for (int b = 0; b < n; b++)
    for (int o = 0; o < oc; o++)
      for (int yy = 0; yy < POS; yy++)
        for (int xx = 0; xx < POS; xx++) {
          double acc = 0;
          for (int i = 0; i < ic; i++)
            for (int ky = 0; ky < k; ky++)
              for (int kx = 0; kx < k; kx++) {
                int sy = yy + ky - pad, sx = xx + kx - pad;
                if (sy < 0 || sy >= POS || sx < 0 || sx >= POS) continue;
                acc += w[(((size_t)o * ic + i) * k + ky) * k + kx] * x[(((size_t)b * ic + i) * POS + sy) * POS + sx];
              }
          y[(((size_t)b * oc + o) * POS + yy) * POS + xx] = acc;
        }
}

// Filter transform G g G^T of a [oc][ic][3][3] filter into the reference's [36][ic][oc] layout, in double.
void kgo_wino_filter_f64(int oc, int ic, const double* w, double* out) {
  for (int o = 0; o < oc; o++)
    for (int i = 0; i < ic; i++) {
      const double* g = w + ((size_t)o * ic + i) * 9;
      double rows[3][6];
      for (int y = 0; y < 3; y++) wino_g(g + 3 * y, rows[y]);
      for (int x = 0; x < 6; x++) {
        double col[3] = {rows[0][x], rows[1][x], rows[2][x]}, t[6];
        wino_g(col, t);
        for (int y = 0; y < 6; y++) out[(((size_t)(y * 6 + x)) * ic + i) * oc + o] = t[y];
      }
    }
}

// The reference's whole Winograd 3x3 convolution in double: tile scatter (t -> n, tile_y, tile_x; window at
// 4*tile - 1, zero outside the 19x19 board), B^T d B, the 36 GEMMs, A^T m A and the crop to the board.
void kgo_conv3x3_winograd_f64(int n, int ic, int oc, const double* x, const double* w, double* y) {
  const int tx = (POS + 3) / 4, ty = (POS + 3) / 4, nt = n * tx * ty;
  std::vector<double> U((size_t)36 * ic * oc), V((size_t)36 * ic * nt), M((size_t)36 * oc * nt, 0.0);
  kgo_wino_filter_f64(oc, ic, w, U.data());
  for (int t = 0; t < nt; t++) {
    const int tile_x = t % tx, tile_y = (t / tx) % ty, b = t / (tx * ty);
    for (int i = 0; i < ic; i++) {
      double d[36], r[36];
      for (int sy = 0; sy < 6; sy++)
        for (int sx = 0; sx < 6; sx++) {
          int yy = tile_y * 4 + sy - 1, xx = tile_x * 4 + sx - 1;
          d[sy * 6 + sx] = (yy >= 0 && yy < POS && xx >= 0 && xx < POS) ? x[(((size_t)b * ic + i) * POS + yy) * POS + xx] : 0.0;
        }
      for (int sy = 0; sy < 6; sy++) wino_bt(d + 6 * sy, r + 6 * sy);
      for (int sx = 0; sx < 6; sx++) {
        double col[6], o[6];
        for (int k = 0; k < 6; k++) col[k] = r[k * 6 + sx];
        wino_bt(col, o);
        for (int k = 0; k < 6; k++) d[k * 6 + sx] = o[k];
      }
      for (int p = 0; p < 36; p++) V[((size_t)p * ic + i) * nt + t] = d[p];
    }
  }
  for (int p = 0; p < 36; p++)
    for (int i = 0; i < ic; i++)
      for (int o = 0; o < oc; o++) {
        const double u = U[((size_t)p * ic + i) * oc + o];
        const double* v = &V[((size_t)p * ic + i) * nt];
        double* mm = &M[((size_t)p * oc + o) * nt];
        for (int t = 0; t < nt; t++) mm[t] += u * v[t];
      }
  for (int t = 0; t < nt; t++) {
    const int tile_x = t % tx, tile_y = (t / tx) % ty, b = t / (tx * ty);
    for (int o = 0; o < oc; o++) {
      double m6[36], r[24];
      for (int p = 0; p < 36; p++) m6[p] = M[((size_t)p * oc + o) * nt + t];
      double rows[6][4];
      for (int sy = 0; sy < 6; sy++) wino_at(m6 + 6 * sy, rows[sy]);
      for (int sx = 0; sx < 4; sx++) {
        double col[6] = {rows[0][sx], rows[1][sx], rows[2][sx], rows[3][sx], rows[4][sx], rows[5][sx]}, o4[4];
        wino_at(col, o4);
        for (int k = 0; k < 4; k++) r[k * 4 + sx] = o4[k];
      }
      for (int sy = 0; sy < 4; sy++)
        for (int sx = 0; sx < 4; sx++) {
          int yy = tile_y * 4 + sy, xx = tile_x * 4 + sx;
          if (yy < POS && xx < POS) y[(((size_t)b * oc + o) * POS + yy) * POS + xx] = r[sy * 4 + sx];
        }
    }
  }
}

// copyWithSymmetry (nninputs.rs:756-850): transpose = bit 2 (square boards only), flipX = bit 1,
// flipY = bit 0; for inputs (reverse = 0) a transpose swaps the two flips.
void kgo_copy_with_symmetry(const float* src, float* dst, int n, int h, int w, int c, int nhwc, int sym, int reverse) {
  const bool transpose = (sym & 4) != 0 && h == w;
  bool fx = (sym & 2) != 0, fy = (sym & 1) != 0;
  if (transpose && !reverse) std::swap(fx, fy);
  for (int b = 0; b < n; b++)
    for (int ch = 0; ch < c; ch++)
      for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++) {
          // The reference moves bases and strides: flipY reverses the destination rows, flipX the
          // destination columns, and a transpose exchanges which source axis walks which.
          const int r = transpose ? x : y, cc = transpose ? y : x;
          const int dy = fy ? h - 1 - r : r;
          const int dx = fx ? w - 1 - cc : cc;
          size_t s, d;
          if (nhwc) {
            s = (((size_t)b * h + y) * w + x) * c + ch;
            d = (((size_t)b * h + dy) * w + dx) * c + ch;
          } else {
            s = (((size_t)b * c + ch) * h + y) * w + x;
            d = (((size_t)b * c + ch) * h + dy) * w + dx;
          }
          dst[d] = src[s];
        }
}

// padded_batch_size (backend.rs:82-84): the smallest bucket in [n, max_batch], else n.
int kgo_padded_batch_size(const int* buckets, int nb, int n, int max_batch) {
  int best = -1;
  for (int k = 0; k < nb; k++)
    if (buckets[k] >= n && buckets[k] <= max_batch && (best < 0 || buckets[k] < best)) best = buckets[k];
  return best < 0 ? n : best;
}

// copy_outputs for one row (backend.rs:650-731): policy optimism mix, inverse symmetry, value/score unpack.
// fields: [win, loss, noresult, score_mean, score_mean_sq, lead, var_time_left, st_winloss_err, st_score_err]
void kgo_copy_outputs_row(const float* row, int P, int S, int version, int sym, float optimism,
                          float* policy_out /*362*/, float* fields /*9*/, float* owner_out /*361 or null*/) {
  const int hw = HW;
  float tmp[HW];
  const float* pol = row;
  if (P == 2 || (P == 4 && version >= 16)) {
    for (int i = 0; i < hw; i++) { float p = pol[i], po = pol[(hw + 1) + i]; tmp[i] = p + (po - p) * optimism; }
    kgo_copy_with_symmetry(tmp, policy_out, 1, POS, POS, 1, 0, sym, 1);
    float p0 = pol[hw], p1 = pol[(hw + 1) + hw];
    policy_out[hw] = p0 + (p1 - p0) * optimism;
  } else {
    kgo_copy_with_symmetry(pol, policy_out, 1, POS, POS, 1, 0, sym, 1);
    policy_out[hw] = pol[hw];
  }
  const float* v = row + P * (hw + 1);
  const float* s = v + 3;
  const float* own = s + S;
  fields[0] = v[0]; fields[1] = v[1]; fields[2] = v[2];
  if (owner_out) kgo_copy_with_symmetry(own, owner_out, 1, POS, POS, 1, 0, sym, 1);
  if (version >= 9) {
    for (int k = 0; k < 6; k++) fields[3 + k] = s[k];
  } else if (version >= 8) {
    fields[3] = s[0]; fields[4] = s[1]; fields[5] = s[2]; fields[6] = s[3]; fields[7] = 0; fields[8] = 0;
  } else if (version >= 4) {
    fields[3] = s[0]; fields[4] = s[1]; fields[5] = s[0]; fields[6] = 0; fields[7] = 0; fields[8] = 0;
  } else {
    fields[3] = s[0]; fields[4] = s[0] * s[0]; fields[5] = s[0]; fields[6] = 0; fields[7] = 0; fields[8] = 0;
  }
}

// NNEvaluator's post-processing of one row's fields (crates/katago-core/src/neuralnet/nneval.rs:1197-1500), after
// kgo_copy_outputs_row: the policy softmax over the legal moves (sequential float sums in position order, as the
// reference), the passing cap (nneval.rs:1247-1258), the uniform fallback, the value softmax and score transforms
// in double by model version (nneval.rs:1298-1477, soft_plus as nneval.rs:1582-1589), and tanh ownership from
// white's perspective with 0 off the board (nneval.rs:1481-1497). The move legality is an input. Returns 0, or
// 1 for a nonfinite policy sum, 2 for a nonfinite value field (the reference's two error returns).
static double kgo_soft_plus(double x) { return x > 40.0 ? x : std::log(1.0 + std::exp(x)); }

int kgo_postprocess_row(const float* row, int P, int S, int version, int sym, float optimism,
                        const unsigned char* legal /*362*/, int white, int bx, int by, float temperature,
                        int passing_hacks, int no_result_allowed, const double* pp /*7*/,
                        float* policy /*362*/, float* fields /*9*/, float* owner /*361*/) {
  float own[HW];
  kgo_copy_outputs_row(row, P, S, version, sym, optimism, policy, fields, own);
  const int n = HW + 1;
  const float scaling = 1.0f / temperature;  // outputScaleMultiplier (1) / nnPolicyTemperature
  float max_policy = -1e25f;
  int legal_count = 0;
  for (int i = 0; i < n; i++) {
    float v;
    if (legal[i]) { legal_count++; v = policy[i] * scaling; }
    else v = -1e30f;
    policy[i] = v;
    if (v > max_policy) max_policy = v;
  }
  if (legal_count == 0) return 4;
  float sum = 0.0f;
  if (passing_hacks) {
    for (int i = 0; i < n - 1; i++) { policy[i] = expf(policy[i] - max_policy); sum += policy[i]; }
    policy[n - 1] = std::max(1e-20f, std::min(expf(policy[n - 1] - max_policy), sum * 19.0f));
    sum += policy[n - 1];
  } else {
    for (int i = 0; i < n; i++) { policy[i] = expf(policy[i] - max_policy); sum += policy[i]; }
  }
  if (!std::isfinite(sum)) return 1;
  if ((double)sum <= 0.0) {
    const float uniform = 1.0f / legal_count;
    for (int i = 0; i < n; i++) policy[i] = legal[i] ? uniform : -1.0f;
  } else {
    for (int i = 0; i < n; i++) policy[i] = legal[i] ? policy[i] / sum : -1.0f;
  }
  const float f_mean = fields[3], f_mean_sq = fields[4], f_lead = fields[5], f_var = fields[6];
  const float f_stw = fields[7], f_sts = fields[8];
  const double win_l = (double)fields[0], loss_l = (double)fields[1];
  double nores_l = (double)fields[2];
  if (version == 3) {
    const double score_value = (double)atanf(f_mean) * 0.63661977236758134308;
    const double mx = std::max(std::max(win_l, loss_l), nores_l);
    double wp = std::exp(win_l - mx), lp = std::exp(loss_l - mx), np = std::exp(nores_l - mx);
    const double ps = wp + lp + np;
    wp /= ps; lp /= ps; np /= ps;
    if (!std::isfinite(ps) || !std::isfinite(score_value)) return 2;
    const double half_pi = 1.57079632679489661923, x = score_value * half_pi;
    const double unscaled = x >= half_pi - 1e-6 ? 1e6 : x <= -half_pi + 1e-6 ? -1e6 : std::tan(x);
    const float sm = (float)(unscaled * (2.0 * std::sqrt((double)bx * (double)by)));
    const float wm = white ? sm : -sm;
    fields[0] = (float)(white ? wp : lp); fields[1] = (float)(white ? lp : wp); fields[2] = (float)np;
    fields[3] = wm; fields[4] = wm * wm; fields[5] = wm; fields[6] = -1.f; fields[7] = -1.f; fields[8] = -1.f;
  } else if (version >= 4) {
    if (!no_result_allowed) nores_l -= 100000.0;
    const double mx = std::max(std::max(win_l, loss_l), nores_l);
    double wp = std::exp(win_l - mx), lp = std::exp(loss_l - mx), np = std::exp(nores_l - mx);
    if (!no_result_allowed) np = 0.0;
    const double ps = wp + lp + np;
    wp /= ps; lp /= ps; np /= ps;
    double mean = (double)f_mean * pp[1];
    const double stdev = kgo_soft_plus((double)f_mean_sq) * pp[2];
    double mean_sq = mean * mean + stdev * stdev;
    double lead = (double)f_lead * pp[3];
    const double var = kgo_soft_plus((double)f_var) * pp[4];
    mean *= 1.0 - np;
    mean_sq *= 1.0 - np;
    lead *= 1.0 - np;
    double stw, sts;
    if (version >= 14) {
      const double a = kgo_soft_plus((double)f_stw * 0.5), b = kgo_soft_plus((double)f_sts * 0.5);
      stw = std::sqrt(a * a * pp[5]);
      sts = std::sqrt(b * b * pp[6]);
    } else if (version >= 10) {
      stw = std::sqrt(kgo_soft_plus((double)f_stw) * pp[5]);
      sts = std::sqrt(kgo_soft_plus((double)f_sts) * pp[6]);
    } else {
      stw = kgo_soft_plus((double)f_stw);
      sts = kgo_soft_plus((double)f_sts) * 10.0;
    }
    if (!std::isfinite(ps) || !std::isfinite(mean) || !std::isfinite(mean_sq) || !std::isfinite(lead) ||
        !std::isfinite(var) || !std::isfinite(stw) || !std::isfinite(sts))
      return 2;
    fields[0] = (float)(white ? wp : lp); fields[1] = (float)(white ? lp : wp); fields[2] = (float)np;
    fields[3] = white ? (float)mean : -(float)mean;
    fields[4] = (float)mean_sq;
    fields[5] = white ? (float)lead : -(float)lead;
    if (version >= 9) { fields[6] = (float)var; fields[7] = (float)stw; fields[8] = (float)sts; }
    else { fields[6] = -1.f; fields[7] = -1.f; fields[8] = -1.f; }
  } else {
    return 3;
  }
  for (int pos = 0; pos < HW; pos++) {
    const int y = pos / POS, x = pos % POS;
    owner[pos] = (y >= by || x >= bx) ? 0.0f : (white ? tanhf(own[pos]) : -tanhf(own[pos]));
  }
  return 0;
}

}  // extern "C"
