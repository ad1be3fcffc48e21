// KataGo model description, parsed from KataGo's model-file format (.bin / .txt, optionally gzip-compressed).
// The structures mirror upstream's desc.h as restated by tools/bin2onnx/bin2onnx.py:141-860; batch norms are
// kept merged (scale / sqrt(var + eps), bias - scale * mean, in float: bin2onnx.py:179-184).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace kgx {

struct ConvDesc {
  std::string name;
  int ky = 0, kx = 0, ic = 0, oc = 0, dy = 1, dx = 1;
  std::vector<float> w;  // [oc][ic][ky][kx]
};

struct BNDesc {
  std::string name;
  int c = 0;
  std::vector<float> scale, bias;  // merged
};

struct MatMulDesc {
  std::string name;
  int ic = 0, oc = 0;
  std::vector<float> w;  // [ic][oc]
};

struct MatBiasDesc {
  std::string name;
  int c = 0;
  std::vector<float> b;
};

enum BlockKind { BLOCK_RES, BLOCK_GPOOL, BLOCK_NBT, BLOCK_ATTN, BLOCK_FFN };

struct BlockDesc {
  BlockKind kind = BLOCK_RES;
  std::string name;
  // Residual / gpool / nested bottleneck: pre BN + act, then `regular` (nbt: the 1x1 pre conv).
  BNDesc pre_bn;
  int pre_act = 0;
  ConvDesc regular;
  // Gpool branch.
  ConvDesc gconv;
  BNDesc gbn;
  int gact = 0;
  MatMulDesc gmul;
  // Mid BN + act (nbt: the post BN + act), then `final_conv` (nbt: the 1x1 post conv).
  BNDesc mid_bn;
  int mid_act = 0;
  ConvDesc final_conv;
  std::vector<BlockDesc> inner;  // nbt
  // Transformer attention.
  int heads = 0, kv_heads = 0, dq = 0, dv = 0;
  bool rope = false, learnable_rope = false;
  float rope_theta = 0.f;
  std::vector<float> rope_freqs;  // [kv_heads][dq/2][2]
  std::vector<float> ln_w;
  float ln_eps = 0.f;
  MatMulDesc q, k, v, o;
  // Transformer FFN.
  int ffn_c = 0;
  bool swiglu = false;
  MatMulDesc l1, lg, l2;
};

struct ModelDesc {
  std::string name;
  int version = 0;
  int num_input_channels = 0, num_global = 0, num_meta = 0, meta_version = 0;
  float post_process[7] = {20.f, 20.f, 20.f, 20.f, 40.f, 0.25f, 30.f};
  int trunk_c = 0, trunk_blocks = 0;
  ConvDesc stem;
  MatMulDesc stem_mm;
  MatMulDesc meta1, meta2, meta3;
  MatBiasDesc meta_b1, meta_b2;
  int meta_act1 = 0, meta_act2 = 0;
  std::vector<BlockDesc> blocks;
  int trunk_norm_kind = 0;  // 0 batch norm, 1 RMSNorm
  BNDesc tip_bn;
  float tip_rms_eps = 0.f;
  bool tip_rms_spatial = false;
  std::vector<float> tip_gamma, tip_beta;
  int tip_act = 0;
  // Policy head.
  int P = 1;
  ConvDesc p1, g1, p2;
  BNDesc g1_bn, p1_bn;
  int g1_act = 0, p1_act = 0;
  MatMulDesc gpool_to_bias, pass1, pass2;
  MatBiasDesc pass_bias;
  int pass_act = 0;
  // Value head.
  ConvDesc v1, own;
  BNDesc v1_bn;
  int v1_act = 0;
  MatMulDesc v2, v3, sv3;
  MatBiasDesc v2_bias, v3_bias, sv3_bias;
  int v2_act = 0;
  int S = 1;

  int row_len() const { return P * (19 * 19 + 1) + 3 + S + 19 * 19; }
  long num_parameters() const;
};

// Parses model-file bytes; throws std::runtime_error with a message naming the offending layer.
ModelDesc parse_model(const uint8_t* data, size_t len);

}  // namespace kgx
