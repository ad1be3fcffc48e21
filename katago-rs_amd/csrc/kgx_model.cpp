// Parser of KataGo's model-file format. Token and check order follow tools/bin2onnx/bin2onnx.py
// (ModelReader :60-125, parse_* :141-860, parse_model :1014-1069), which mirrors upstream desc.cpp.
#include "kgx_model.h"

#include <zlib.h>

#include <cctype>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace kgx {
namespace {

struct Reader {
  const uint8_t* d;
  size_t n;
  size_t pos;
  bool binary_floats;

  static bool is_ws(uint8_t c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\v' || c == '\f'; }
  void skip_ws() {
    while (pos < n && is_ws(d[pos])) pos++;
  }
  std::string token() {
    skip_ws();
    const size_t start = pos;
    while (pos < n && !is_ws(d[pos])) pos++;
    if (pos == start) throw std::runtime_error("Unexpected end of model file");
    return std::string(reinterpret_cast<const char*>(d + start), pos - start);
  }
  int integer() {
    const std::string t = token();
    char* end = nullptr;
    const long v = std::strtol(t.c_str(), &end, 10);
    if (end == t.c_str() || *end != '\0') throw std::runtime_error("Expected an integer but got " + t);
    return static_cast<int>(v);
  }
  float real() {
    const std::string t = token();
    char* end = nullptr;
    const float v = std::strtof(t.c_str(), &end);
    if (end == t.c_str() || *end != '\0') throw std::runtime_error("Expected a float but got " + t);
    return v;
  }
  bool boolean() {
    const int v = integer();
    if (v != 0 && v != 1) throw std::runtime_error("Expected bool 0/1 but got " + std::to_string(v));
    return v == 1;
  }
  std::vector<float> floats(size_t count, const std::string& name) {
    std::vector<float> out(count);
    if (!binary_floats) {
      for (size_t k = 0; k < count; k++) out[k] = real();
    } else {
      // "@BIN@" then count little-endian floats, at most 100 bytes after the previous token.
      int before = 0;
      for (;;) {
        if (pos >= n) throw std::runtime_error(name + ": could not find binary float block");
        const uint8_t c = d[pos++];
        if (c == '@') break;
        if (++before > 100) throw std::runtime_error(name + ": could not read float weights (no @BIN@ header)");
      }
      if (pos + 4 > n || std::memcmp(d + pos, "BIN@", 4) != 0)
        throw std::runtime_error(name + ": did not find expected header for binary float block");
      pos += 4;
      if (pos + 4 * count > n)
        throw std::runtime_error(name + ": did not find the expected number of floats in binary float block");
      std::memcpy(out.data(), d + pos, 4 * count);
      pos += 4 * count;
    }
    for (float v : out)
      if (!std::isfinite(v)) throw std::runtime_error(name + ": Nan or infinite neural net weight or parameter");
    return out;
  }
};

void require(bool cond, const std::string& msg) {
  if (!cond) throw std::runtime_error(msg);
}

ConvDesc parse_conv(Reader& r) {
  ConvDesc c;
  c.name = r.token();
  c.ky = r.integer(); c.kx = r.integer(); c.ic = r.integer(); c.oc = r.integer();
  c.dy = r.integer(); c.dx = r.integer();
  require(c.kx > 0 && c.ky > 0, c.name + ": convolution filter sizes must be positive");
  require(c.ic > 0 && c.oc > 0, c.name + ": number of in and out channels must be positive");
  require(c.dx > 0 && c.dy > 0, c.name + ": dilation factors must be positive");
  require(c.kx % 2 == 1 && c.ky % 2 == 1, c.name + ": convolution filter sizes must be odd");
  const std::vector<float> raw = r.floats((size_t)c.ky * c.kx * c.ic * c.oc, c.name);
  c.w.resize(raw.size());
  for (int y = 0; y < c.ky; y++)
    for (int x = 0; x < c.kx; x++)
      for (int i = 0; i < c.ic; i++)
        for (int o = 0; o < c.oc; o++)
          c.w[(((size_t)o * c.ic + i) * c.ky + y) * c.kx + x] = raw[(((size_t)y * c.kx + x) * c.ic + i) * c.oc + o];
  return c;
}

BNDesc parse_bn(Reader& r) {
  BNDesc b;
  b.name = r.token();
  b.c = r.integer();
  const float eps = r.real();
  const bool has_scale = r.boolean();
  const bool has_bias = r.boolean();
  require(b.c >= 1, b.name + ": numChannels < 1");
  require(eps > 0 && std::isfinite(eps), b.name + ": epsilon is not positive and finite");
  const std::vector<float> mean = r.floats(b.c, b.name);
  const std::vector<float> var = r.floats(b.c, b.name);
  const std::vector<float> scale = has_scale ? r.floats(b.c, b.name) : std::vector<float>(b.c, 1.0f);
  const std::vector<float> bias = has_bias ? r.floats(b.c, b.name) : std::vector<float>(b.c, 0.0f);
  b.scale.resize(b.c);
  b.bias.resize(b.c);
  for (int i = 0; i < b.c; i++) {
    const float s = scale[i] / std::sqrt(var[i] + eps);
    b.scale[i] = s;
    b.bias[i] = bias[i] - s * mean[i];
  }
  return b;
}

int parse_act(Reader& r, int version) {
  const std::string name = r.token();
  if (version < 11) return 1;  // relu
  const std::string kind = r.token();
  if (kind == "ACTIVATION_IDENTITY") return 0;
  if (kind == "ACTIVATION_RELU") return 1;
  if (kind == "ACTIVATION_MISH") return 2;
  if (kind == "ACTIVATION_SILU") return 3;
  throw std::runtime_error(name + ": unknown activation " + kind);
}

MatMulDesc parse_matmul(Reader& r) {
  MatMulDesc m;
  m.name = r.token();
  m.ic = r.integer();
  m.oc = r.integer();
  require(m.ic > 0 && m.oc > 0, m.name + ": number of in and out channels must be positive");
  m.w = r.floats((size_t)m.ic * m.oc, m.name);
  return m;
}

MatBiasDesc parse_matbias(Reader& r) {
  MatBiasDesc b;
  b.name = r.token();
  b.c = r.integer();
  require(b.c > 0, b.name + ": number of channels must be positive");
  b.b = r.floats(b.c, b.name);
  return b;
}

void parse_tf_rmsnorm(Reader& r, BlockDesc& b) {
  const std::string name = r.token();
  const int c = r.integer();
  b.ln_eps = r.real();
  require(c >= 1, name + ": transformer rmsnorm numChannels < 1");
  require(b.ln_eps > 0 && b.ln_eps <= 1.0f, name + ": transformer rmsnorm epsilon is not positive or is too large");
  b.ln_w = r.floats(c, name);
}

std::vector<BlockDesc> parse_stack(Reader& r, int version, const std::string& name, int num_blocks, int trunk_c);

BlockDesc parse_block(Reader& r, int version, const std::string& kind) {
  BlockDesc b;
  if (kind == "ordinary_block") {
    b.kind = BLOCK_RES;
    b.name = r.token();
    b.pre_bn = parse_bn(r); b.pre_act = parse_act(r, version);
    b.regular = parse_conv(r);
    b.mid_bn = parse_bn(r); b.mid_act = parse_act(r, version);
    b.final_conv = parse_conv(r);
    require(b.pre_bn.c == b.regular.ic, b.name + ": preBN.numChannels != regularConv.inChannels");
    require(b.mid_bn.c == b.regular.oc, b.name + ": midBN.numChannels != regularConv.outChannels");
    require(b.mid_bn.c == b.final_conv.ic, b.name + ": midBN.numChannels != finalConv.inChannels");
  } else if (kind == "gpool_block") {
    b.kind = BLOCK_GPOOL;
    b.name = r.token();
    b.pre_bn = parse_bn(r); b.pre_act = parse_act(r, version);
    b.regular = parse_conv(r);
    b.gconv = parse_conv(r);
    b.gbn = parse_bn(r); b.gact = parse_act(r, version);
    b.gmul = parse_matmul(r);
    b.mid_bn = parse_bn(r); b.mid_act = parse_act(r, version);
    b.final_conv = parse_conv(r);
    require(b.pre_bn.c == b.regular.ic, b.name + ": preBN.numChannels != regularConv.inChannels");
    require(b.pre_bn.c == b.gconv.ic, b.name + ": preBN.numChannels != gpoolConv.inChannels");
    require(b.gbn.c == b.gconv.oc, b.name + ": gpoolBN.numChannels != gpoolConv.outChannels");
    require(b.gbn.c * 3 == b.gmul.ic, b.name + ": gpoolBN.numChannels*3 != gpoolToBiasMul.inChannels");
    require(b.mid_bn.c == b.regular.oc, b.name + ": midBN.numChannels != regularConv.outChannels");
    require(b.mid_bn.c == b.gmul.oc, b.name + ": midBN.numChannels != gpoolToBiasMul.outChannels");
    require(b.mid_bn.c == b.final_conv.ic, b.name + ": midBN.numChannels != finalConv.inChannels");
  } else if (kind == "nested_bottleneck_block") {
    b.kind = BLOCK_NBT;
    b.name = r.token();
    const int num_blocks = r.integer();
    require(num_blocks >= 1, b.name + ": nested bottleneck res block num blocks must be positive");
    b.pre_bn = parse_bn(r); b.pre_act = parse_act(r, version);
    b.regular = parse_conv(r);
    b.inner = parse_stack(r, version, b.name, num_blocks, b.regular.oc);
    b.mid_bn = parse_bn(r); b.mid_act = parse_act(r, version);
    b.final_conv = parse_conv(r);
    require(b.pre_bn.c == b.regular.ic, b.name + ": preBN.numChannels != preConv.inChannels");
    require(b.mid_bn.c == b.regular.oc, b.name + ": postBN.numChannels != preConv.outChannels");
    require(b.mid_bn.c == b.final_conv.ic, b.name + ": postBN.numChannels != postConv.inChannels");
  } else if (kind == "transformer_attention_block") {
    b.kind = BLOCK_ATTN;
    b.name = r.token();
    b.heads = r.integer(); b.kv_heads = r.integer(); b.dq = r.integer(); b.dv = r.integer();
    b.rope = r.integer() != 0;
    b.learnable_rope = r.integer() != 0;
    require(b.heads >= 1 && b.kv_heads >= 1, b.name + ": transformer attention numHeads and numKVHeads must be positive");
    require(b.heads % b.kv_heads == 0, b.name + ": numHeads must be divisible by numKVHeads");
    require(b.dq >= 1 && b.dv >= 1, b.name + ": head dims must be positive");
    require(!b.rope || b.dq % 2 == 0, b.name + ": qHeadDim must be even when RoPE is used");
    parse_tf_rmsnorm(r, b);
    b.q = parse_matmul(r); b.k = parse_matmul(r); b.v = parse_matmul(r); b.o = parse_matmul(r);
    require(b.q.oc == b.heads * b.dq, b.name + ": qProj.outChannels != numHeads*qHeadDim");
    require(b.k.oc == b.kv_heads * b.dq, b.name + ": kProj.outChannels != numKVHeads*qHeadDim");
    require(b.v.oc == b.kv_heads * b.dv, b.name + ": vProj.outChannels != numKVHeads*vHeadDim");
    require(b.o.ic == b.heads * b.dv, b.name + ": outProj.inChannels != numHeads*vHeadDim");
    if (b.rope) {
      r.token();
      if (b.learnable_rope) {
        const int nkv = r.integer(), npairs = r.integer(), dim2 = r.integer();
        require(nkv == b.kv_heads, b.name + ": ropeNumKVHeads != numKVHeads");
        require(npairs == b.dq / 2, b.name + ": ropeNumPairs != qHeadDim/2");
        require(dim2 == 2, b.name + ": rope freq dim2 must be 2");
        b.rope_freqs = r.floats((size_t)nkv * npairs * 2, b.name);
      } else {
        b.rope_theta = r.real();
        require(b.rope_theta > 0 && std::isfinite(b.rope_theta), b.name + ": rope theta must be positive and finite");
      }
    }
  } else if (kind == "transformer_ffn_block") {
    b.kind = BLOCK_FFN;
    b.name = r.token();
    const int c = r.integer();
    b.ffn_c = r.integer();
    b.swiglu = r.integer() != 0;
    require(c >= 1 && b.ffn_c >= 1, b.name + ": transformer ffn channels must be positive");
    parse_tf_rmsnorm(r, b);
    b.l1 = parse_matmul(r);
    if (b.swiglu) b.lg = parse_matmul(r);
    b.l2 = parse_matmul(r);
    require(b.l1.ic == c && b.l1.oc == b.ffn_c, b.name + ": linear1 shape != (numChannels, ffnChannels)");
    if (b.swiglu) require(b.lg.ic == c && b.lg.oc == b.ffn_c, b.name + ": linearGate shape != (numChannels, ffnChannels)");
    require(b.l2.ic == b.ffn_c && b.l2.oc == c, b.name + ": linear2 shape != (ffnChannels, numChannels)");
    b.pre_bn.c = c;
  } else {
    throw std::runtime_error("found unknown block kind " + kind);
  }
  return b;
}

int block_in_channels(const BlockDesc& b) {
  switch (b.kind) {
    case BLOCK_ATTN: return b.q.ic;
    case BLOCK_FFN: return b.l1.ic;
    default: return b.pre_bn.c;
  }
}

int block_out_channels(const BlockDesc& b) {
  switch (b.kind) {
    case BLOCK_ATTN: return b.o.oc;
    case BLOCK_FFN: return b.l2.oc;
    default: return b.final_conv.oc;
  }
}

std::vector<BlockDesc> parse_stack(Reader& r, int version, const std::string& name, int num_blocks, int trunk_c) {
  std::vector<BlockDesc> out;
  for (int i = 0; i < num_blocks; i++) {
    const std::string kind = r.token();
    BlockDesc b = parse_block(r, version, kind);
    require(block_in_channels(b) == trunk_c, name + ": " + b.name + " input channels != trunk channels");
    require(block_out_channels(b) == trunk_c, name + ": " + b.name + " output channels != trunk channels");
    out.push_back(std::move(b));
  }
  return out;
}

void check_name_valid(const std::string& name) {
  require(!name.empty() && name.size() <= 96, "Model name must be 1..96 chars: " + name);
  for (char c : name)
    require(std::isalnum((unsigned char)c) || c == '_' || c == '-',
            "Model name must contain only alphanumeric characters, underscores, and hyphens: " + name);
}

bool gunzip(const uint8_t* d, size_t n, std::vector<uint8_t>& out) {
  if (n < 2 || d[0] != 0x1f || d[1] != 0x8b) return false;
  z_stream zs;
  std::memset(&zs, 0, sizeof(zs));
  if (inflateInit2(&zs, 15 + 32) != Z_OK) throw std::runtime_error("Error loading model file: zlib init failed");
  zs.next_in = const_cast<uint8_t*>(d);
  zs.avail_in = static_cast<uInt>(n);
  std::vector<uint8_t> chunk(1 << 20);
  int rc;
  do {
    zs.next_out = chunk.data();
    zs.avail_out = static_cast<uInt>(chunk.size());
    rc = inflate(&zs, Z_NO_FLUSH);
    if (rc != Z_OK && rc != Z_STREAM_END) {
      inflateEnd(&zs);
      throw std::runtime_error("Error loading model file: corrupt gzip data");
    }
    out.insert(out.end(), chunk.data(), chunk.data() + (chunk.size() - zs.avail_out));
  } while (rc != Z_STREAM_END);
  inflateEnd(&zs);
  return true;
}

}  // namespace

long ModelDesc::num_parameters() const {
  long n = 0;
  auto conv = [&](const ConvDesc& c) { n += (long)c.w.size(); };
  auto mm = [&](const MatMulDesc& m) { n += (long)m.w.size(); };
  auto bn = [&](const BNDesc& b) { n += 2L * b.c; };
  std::vector<const std::vector<BlockDesc>*> todo{&blocks};
  while (!todo.empty()) {
    const std::vector<BlockDesc>* bs = todo.back();
    todo.pop_back();
    for (const BlockDesc& b : *bs) {
      if (b.kind == BLOCK_ATTN) {
        n += (long)b.ln_w.size() + (long)b.rope_freqs.size();
        mm(b.q); mm(b.k); mm(b.v); mm(b.o);
      } else if (b.kind == BLOCK_FFN) {
        n += (long)b.ln_w.size();
        mm(b.l1); mm(b.lg); mm(b.l2);
      } else {
        bn(b.pre_bn); conv(b.regular); bn(b.mid_bn); conv(b.final_conv);
        if (b.kind == BLOCK_GPOOL) { conv(b.gconv); bn(b.gbn); mm(b.gmul); }
        if (b.kind == BLOCK_NBT) todo.push_back(&b.inner);
      }
    }
  }
  conv(stem); mm(stem_mm);
  conv(p1); conv(g1); conv(p2); bn(g1_bn); bn(p1_bn); mm(gpool_to_bias); mm(pass1); mm(pass2);
  conv(v1); conv(own); bn(v1_bn); mm(v2); mm(v3); mm(sv3);
  return n;
}

ModelDesc parse_model(const uint8_t* data, size_t len) {
  std::vector<uint8_t> inflated;
  if (gunzip(data, len, inflated)) {
    data = inflated.data();
    len = inflated.size();
  }
  // Binary-float files carry "@BIN@" blocks; a text file cannot contain '@'.
  bool binary = false;
  for (size_t k = 0; k + 5 <= len; k++)
    if (data[k] == '@' && std::memcmp(data + k, "@BIN@", 5) == 0) { binary = true; break; }
  Reader r{data, len, 0, binary};

  ModelDesc m;
  m.name = r.token();
  m.version = r.integer();
  check_name_valid(m.name);
  require(m.version >= 3, m.name + ": model version " + std::to_string(m.version) + " is too old");
  require(m.version <= 17, "This neural net requires a newer KataGo version. Model version: " + std::to_string(m.version));
  m.num_input_channels = r.integer();
  require(m.num_input_channels > 0, m.name + ": numInputChannels must be positive");
  m.num_global = r.integer();
  require(m.num_global > 0, m.name + ": numInputGlobalChannels must be positive");
  if (m.version >= 13) {
    for (int k = 0; k < 7; k++) {
      m.post_process[k] = r.real();
      require(m.post_process[k] > 0, m.name + ": post-process params must be positive");
    }
  }
  if (m.version >= 15) {
    m.meta_version = r.integer();
    require(m.meta_version == 0 || m.meta_version == 1, m.name + ": unsupported metaEncoderVersion");
    m.num_meta = m.meta_version == 1 ? 192 : 0;
    for (int k = 0; k < 2; k++) {
      const int v = r.integer();
      require(v == 0 || v == 1, m.name + ": model flag unexpected value");
    }
    for (int k = 0; k < 5; k++) require(r.integer() == 0, m.name + ": unknown/unsupported model option");
  }
  // Trunk (bin2onnx.py:691-741).
  const std::string trunk_name = r.token();
  m.trunk_blocks = r.integer();
  m.trunk_c = r.integer();
  const int mid_c = r.integer(), regular_c = r.integer();
  r.integer();  // dilated channels, unused
  const int gpool_c = r.integer();
  if (m.version >= 15) {
    m.trunk_norm_kind = r.integer();
    for (int k = 0; k < 5; k++) require(r.integer() == 0, trunk_name + ": unknown/unsupported trunk option");
    require(m.trunk_norm_kind == 0 || m.trunk_norm_kind == 1, trunk_name + ": unknown or unsupported trunk norm kind");
  }
  require(m.trunk_blocks >= 1, trunk_name + ": trunk num blocks must be positive");
  require(m.trunk_c > 0 && mid_c > 0 && regular_c > 0 && gpool_c > 0, trunk_name + ": channel counts must be positive");
  m.stem = parse_conv(r);
  require(m.stem.oc == m.trunk_c, m.stem.name + ": outChannels != trunkNumChannels");
  m.stem_mm = parse_matmul(r);
  require(m.stem_mm.oc == m.trunk_c, m.stem_mm.name + ": outChannels != trunkNumChannels");
  if (m.meta_version > 0) {
    const std::string enc = r.token();
    require(r.integer() == 192, enc + ": number of in channels did not match expected (192)");
    m.meta1 = parse_matmul(r); m.meta_b1 = parse_matbias(r); m.meta_act1 = parse_act(r, m.version);
    m.meta2 = parse_matmul(r); m.meta_b2 = parse_matbias(r); m.meta_act2 = parse_act(r, m.version);
    m.meta3 = parse_matmul(r);
    require(m.meta1.ic == 192 && m.meta1.oc == m.meta_b1.c && m.meta2.ic == m.meta1.oc && m.meta2.oc == m.meta_b2.c &&
                m.meta3.ic == m.meta2.oc && m.meta3.oc == m.trunk_c,
            enc + ": SGF metadata encoder shapes do not chain");
  }
  m.blocks = parse_stack(r, m.version, trunk_name, m.trunk_blocks, m.trunk_c);
  if (m.trunk_norm_kind == 0) {
    m.tip_bn = parse_bn(r);
    require(m.tip_bn.c == m.trunk_c, trunk_name + ": trunkTipBN.numChannels != trunkNumChannels");
  } else {
    const std::string name = r.token();
    const int c = r.integer();
    m.tip_rms_eps = r.real();
    m.tip_rms_spatial = r.integer() != 0;
    const int cgroup = r.integer();
    require(m.tip_rms_eps > 0 && m.tip_rms_eps <= 1.0f, name + ": rmsnorm epsilon is not positive or is too large");
    require(c == m.trunk_c, trunk_name + ": trunkTipRMSNorm.numChannels != trunkNumChannels");
    require(cgroup == 0, name + ": grouped spatial RMSNorm is not supported");
    m.tip_gamma = r.floats(c, name);
    m.tip_beta = r.floats(c, name);
  }
  m.tip_act = parse_act(r, m.version);
  // Policy head (bin2onnx.py:762-811).
  const std::string ph = r.token();
  if (m.version >= 17) {
    m.P = r.integer();
    require(m.P == 2 || m.P == 4, ph + ": policy head got invalid policyOutChannels");
    for (int k = 0; k < 3; k++) require(r.integer() == 0, ph + ": unknown/unsupported policy option");
  } else if (m.version == 16) {
    m.P = 4;
  } else if (m.version >= 12) {
    m.P = 2;
  } else {
    m.P = 1;
  }
  m.p1 = parse_conv(r);
  m.g1 = parse_conv(r);
  m.g1_bn = parse_bn(r); m.g1_act = parse_act(r, m.version);
  m.gpool_to_bias = parse_matmul(r);
  m.p1_bn = parse_bn(r); m.p1_act = parse_act(r, m.version);
  m.p2 = parse_conv(r);
  m.pass1 = parse_matmul(r);
  if (m.version >= 15) {
    m.pass_bias = parse_matbias(r);
    m.pass_act = parse_act(r, m.version);
    m.pass2 = parse_matmul(r);
  }
  require(m.p1.oc == m.p1_bn.c, ph + ": p1Conv.outChannels != p1BN.numChannels");
  require(m.g1.oc == m.g1_bn.c, ph + ": g1Conv.outChannels != g1BN.numChannels");
  require(m.gpool_to_bias.ic == m.g1_bn.c * 3, ph + ": gpoolToBiasMul.inChannels != g1BN.numChannels*3");
  require(m.gpool_to_bias.oc == m.p1_bn.c, ph + ": gpoolToBiasMul.outChannels != p1BN.numChannels");
  require(m.p2.ic == m.p1_bn.c, ph + ": p2Conv.inChannels != p1BN.numChannels");
  require(m.pass1.ic == m.g1_bn.c * 3, ph + ": gpoolToPassMul.inChannels != g1BN.numChannels*3");
  require(m.p2.oc == m.P, ph + ": p2Conv.outChannels != policyOutChannels");
  if (m.version >= 15) {
    require(m.pass1.oc == m.pass_bias.c && m.pass1.oc == m.pass2.ic && m.pass2.oc == m.P, ph + ": pass head shapes do not chain");
  } else {
    require(m.pass1.oc == m.P, ph + ": gpoolToPassMul.outChannels != policyOutChannels");
  }
  // Value head (bin2onnx.py:829-860).
  const std::string vh = r.token();
  if (m.version >= 17)
    for (int k = 0; k < 3; k++) require(r.integer() == 0, vh + ": unknown/unsupported value option");
  m.v1 = parse_conv(r); m.v1_bn = parse_bn(r); m.v1_act = parse_act(r, m.version);
  m.v2 = parse_matmul(r); m.v2_bias = parse_matbias(r); m.v2_act = parse_act(r, m.version);
  m.v3 = parse_matmul(r); m.v3_bias = parse_matbias(r);
  m.sv3 = parse_matmul(r); m.sv3_bias = parse_matbias(r);
  m.own = parse_conv(r);
  require(m.v1.oc == m.v1_bn.c, vh + ": v1Conv.outChannels != v1BN.numChannels");
  require(m.v2.ic == m.v1_bn.c * 3, vh + ": v2Mul.inChannels != v1BN.numChannels*3");
  require(m.v2.oc == m.v2_bias.c && m.v2.oc == m.v3.ic && m.v2.oc == m.sv3.ic, vh + ": v2 shapes do not chain");
  require(m.v3.oc == 3 && m.v3_bias.c == 3, vh + ": v3 must have 3 outputs");
  const int expected_sv = m.version >= 9 ? 6 : m.version >= 8 ? 4 : m.version >= 4 ? 2 : 1;
  require(m.sv3.oc == expected_sv && m.sv3_bias.c == expected_sv, vh + ": sv3 has the wrong number of outputs for its model version");
  require(m.own.ic == m.v1.oc && m.own.oc == 1, vh + ": vOwnershipConv shape");
  m.S = m.sv3.oc;
  require(m.num_input_channels == m.stem.ic, m.name + ": numInputChannels != initialConv.inChannels");
  require(m.num_global == m.stem_mm.ic, m.name + ": numInputGlobalChannels != initialMatMul.inChannels");
  require(m.trunk_c == m.p1.ic && m.trunk_c == m.g1.ic && m.trunk_c == m.v1.ic, m.name + ": trunk channels != head input channels");
  r.skip_ws();
  require(r.pos == r.n, m.name + ": " + std::to_string(r.n - r.pos) + " unparsed trailing bytes in model file");
  return m;
}

}  // namespace kgx
