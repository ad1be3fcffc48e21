"""Seeded synthetic KataGo networks and inputs.

Writes networks in KataGo's own model-file format (the ``.bin`` format: whitespace-separated header
tokens, weights as ``@BIN@`` blocks of little-endian float32), which is what the loader of this library
parses. The token order per layer and block follows the parser of tools/bin2onnx/bin2onnx.py
(parse_conv :141-158, parse_bn :187-200, parse_activation :208-215, parse_matmul :226-234,
parse_residual_block :275-288, parse_gpool_block :312-333, parse_nested_bottleneck_block :354-370,
parse_rmsnorm :384-396, parse_transformer_rmsnorm :407-413, parse_transformer_attention :491-520,
parse_transformer_ffn :542-560, parse_trunk :691-741, parse_policy_head :762-811,
parse_value_head :829-860, parse_model :1014-1069).

Weight distributions are the benchmark's: He-normal convolutions (sigma = sqrt(2 / fan_in)), batch norm
gamma ~ U(0.8, 1.2), beta ~ N(0, 0.1), running mean ~ N(0, 0.1), running var ~ U(0.5, 1.5), eps 1e-5;
matmuls and transformer linears N(0, 1/sqrt(fan_in)); RMSNorm gains ~ U(0.9, 1.1). One departure: the
last layer of every residual branch (the final conv of a residual/gpool block, the post conv of a nested
bottleneck block, the out projection and second FFN linear of a transformer block) is scaled by
1/sqrt(L), L the number of residual additions into the same stream (Fixup, Zhang et al. 2019). Without it
the seeded b18c384nbt trunk grows about 2.5x per block (std 1.7e7 after 18 blocks), beyond float16's
range, so no half-precision result could be compared with anything.

Random numbers come from numpy's PCG64 generator (``numpy.random.default_rng(seed)``), drawn in file order.
"""

from __future__ import annotations

import io
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

POS_LEN = 19
HW = POS_LEN * POS_LEN


# ---------------------------------------------------------------------------------------------------------------
# Architecture descriptions
# ---------------------------------------------------------------------------------------------------------------

@dataclass
class Arch:
    name: str
    model_version: int
    trunk_c: int
    blocks: list                       # list of block specs (tuples, see below)
    num_input_channels: int = 22
    num_global_channels: int = 19
    p1_c: int = 32
    g1_c: int = 32
    v1_c: int = 32
    v2_c: int = 64
    stem_k: int = 3
    mid_c: int = 0                     # header fields only
    gpool_c: int = 32
    act: str = "ACTIVATION_MISH"
    tip: str = "bn"                    # "bn" | "rms" | "rms_spatial"
    meta_encoder: int = 0              # 0 or 1 (192 meta channels)
    meta_c: int = 64                   # meta encoder hidden width
    policy_channels: int = 0           # v17 only (2 or 4); derived otherwise
    rope_theta: float = 100.0
    qk_gain: float = 1.0               # scale of the attention q and k projections (scores scale by its square)
    mid_bn_gain: float = 1.0           # scale of ordinary residual blocks' mid batch-norm gamma and beta


# Block specs:
#   ("res", c_mid)                                      ordinary residual block, 3x3 convs
#   ("gpool", c_regular, c_gpool)                       global pooling residual block
#   ("nbt", c_inner, [inner block specs])               nested bottleneck block (1x1 in/out)
#   ("attn", heads, kv_heads, dq, dv, rope)             rope: "fixed" | "learnable" | "none"
#   ("ffn", ffn_c, swiglu)

def _nbt_b18(gpool: bool):
    inner1 = ("gpool", 192, 64) if gpool else ("res", 192)
    return ("nbt", 192, [inner1, ("res", 192)])


def cfg_b10c128() -> Arch:
    blocks = [("gpool", 128, 32) if i % 3 == 2 else ("res", 128) for i in range(10)]
    return Arch("b10c128", 14, 128, blocks, mid_c=128, gpool_c=32)


def cfg_b18c384nbt() -> Arch:
    blocks = [_nbt_b18(i % 3 == 2) for i in range(18)]
    return Arch("b18c384nbt", 14, 384, blocks, mid_c=192, gpool_c=64)


def _tf_blocks(n, heads, dq, ffn_c, swiglu, kv_heads=None, rope="fixed"):
    kv = heads if kv_heads is None else kv_heads
    out = []
    for _ in range(n):
        out.append(("attn", heads, kv, dq, dq, rope))
        out.append(("ffn", ffn_c, swiglu))
    return out


def cfg_b10c384h6() -> Arch:
    return Arch("b10c384h6", 15, 384, _tf_blocks(10, 6, 64, 1536, False), mid_c=384)


def cfg_b10c512h8() -> Arch:
    return Arch("b10c512h8", 15, 512, _tf_blocks(10, 8, 64, 2048, True), mid_c=512)


def cfg_tf3_b11c768() -> Arch:
    return Arch("tf3-b11c768", 15, 768, _tf_blocks(11, 12, 64, 3072, True), mid_c=768)


# The benchmark workloads: (architecture, batch size).
CONFIGS = {
    "b10c128": (cfg_b10c128, 8),
    "b18c384nbt": (cfg_b18c384nbt, 32),
    "b10c384h6": (cfg_b10c384h6, 32),
    "b10c512h8": (cfg_b10c512h8, 64),
    "tf3-b11c768": (cfg_tf3_b11c768, 64),
}
CONFIG_SEEDS = {
    "b10c128": 0x6B67000000000000,
    "b18c384nbt": 0x6B67000000000001,
    "b10c384h6": 0x6B67000000000002,
    "b10c512h8": 0x6B67000000000003,
    "tf3-b11c768": 0x6B67000000000004,
}


# Small nets for parity tests: every block kind, head variant and model-version branch at sizes the CPU
# oracle runs in well under a second.
def tiny_nets() -> dict:
    return {
        "t_res": Arch("t-res", 14, 32, [("res", 32), ("gpool", 32, 16), ("res", 32)], gpool_c=16,
                      p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_nbt": Arch("t-nbt", 14, 64, [("nbt", 32, [("gpool", 32, 16), ("res", 32)]),
                                        ("nbt", 32, [("res", 32), ("res", 32)])],
                      mid_c=32, gpool_c=16, p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_v8": Arch("t-v8", 8, 32, [("res", 32), ("gpool", 32, 16)], stem_k=5, act="ACTIVATION_RELU",
                     gpool_c=16, p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_tf": Arch("t-tf", 15, 64, [("attn", 2, 2, 32, 32, "fixed"), ("ffn", 128, True),
                                      ("attn", 4, 2, 16, 16, "learnable"), ("ffn", 96, False)],
                     p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_tf64": Arch("t-tf64", 15, 96, [("attn", 2, 1, 64, 64, "fixed"), ("ffn", 128, True),
                                          ("attn", 2, 2, 64, 64, "none"), ("ffn", 96, True)],
                       p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_human": Arch("t-human", 15, 32, [("res", 32), ("gpool", 32, 16)], meta_encoder=1, meta_c=32,
                        gpool_c=16, p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_rms": Arch("t-rms", 17, 64, [("nbt", 32, [("attn", 2, 2, 16, 16, "fixed"), ("ffn", 64, True)]),
                                        ("res", 64)],
                      tip="rms_spatial", act="ACTIVATION_SILU", policy_channels=4,
                      p1_c=16, g1_c=16, v1_c=16, v2_c=24),
        "t_rmspos": Arch("t-rmspos", 17, 32, [("res", 32)], tip="rms", policy_channels=2,
                         p1_c=16, g1_c=16, v1_c=16, v2_c=24),
    }


def num_policy_channels(arch: Arch) -> int:
    """PolicyHeadDesc's policyOutChannels by model version (bin2onnx.py:762-776)."""
    v = arch.model_version
    if v >= 17:
        return arch.policy_channels or 2
    if v == 16:
        return 4
    if v >= 12:
        return 2
    return 1


def num_score_channels(arch: Arch) -> int:
    """ValueHeadDesc's expected sv3 outputs by model version (bin2onnx.py:849-856)."""
    v = arch.model_version
    if v >= 9:
        return 6
    if v >= 8:
        return 4
    if v >= 4:
        return 2
    return 1


def row_len(arch: Arch) -> int:
    """Floats per batch row of the readback: policy P*(HW+1), value 3, score S, ownership HW."""
    return num_policy_channels(arch) * (HW + 1) + 3 + num_score_channels(arch) + HW


# ---------------------------------------------------------------------------------------------------------------
# Writer
# ---------------------------------------------------------------------------------------------------------------

class _Writer:
    def __init__(self, rng: np.random.Generator, model_version: int, text_floats: bool = False):
        self.buf = io.BytesIO()
        self.rng = rng
        self.v = model_version
        self.text = text_floats
        self._n = 0

    def name(self, base: str) -> str:
        self._n += 1
        return f"{base}{self._n}"

    def tok(self, *items):
        for it in items:
            if isinstance(it, float):
                it = repr(float(np.float32(it)))
            self.buf.write(str(it).encode("ascii"))
            self.buf.write(b"\n")

    def floats(self, arr: np.ndarray):
        if self.text:
            vals = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
            self.buf.write(" ".join(repr(float(x)) for x in vals).encode("ascii"))
            self.buf.write(b"\n")
            return
        self.buf.write(b"@BIN@")
        self.buf.write(np.ascontiguousarray(arr, dtype="<f4").tobytes())
        self.buf.write(b"\n")

    # --- layers ---
    def conv(self, base, k, ic, oc, gain=1.0, zero=False):
        self.tok(self.name(base), k, k, ic, oc, 1, 1)
        std = np.sqrt(2.0 / (ic * k * k)) * gain
        w = self.rng.normal(0.0, std, size=(oc, ic, k, k)).astype(np.float32)
        if zero:
            w[:] = 0
        # File order is y, x, ic, oc.
        self.floats(w.transpose(2, 3, 1, 0))
        return w

    def bn(self, base, c, gain=1.0):
        self.tok(self.name(base), c, 1e-5, 1, 1)
        mean = self.rng.normal(0.0, 0.1, c)
        var = self.rng.uniform(0.5, 1.5, c)
        gamma = self.rng.uniform(0.8, 1.2, c) * gain
        beta = self.rng.normal(0.0, 0.1, c) * gain
        self.floats(mean)
        self.floats(var)
        self.floats(gamma)
        self.floats(beta)
        f = np.float32
        return {"mean": mean.astype(f), "var": var.astype(f), "gamma": gamma.astype(f), "beta": beta.astype(f),
                "eps": f(1e-5)}

    def act(self, base, kind):
        self.tok(self.name(base))
        if self.v >= 11:
            self.tok(kind)
        return kind if self.v >= 11 else "ACTIVATION_RELU"

    def matmul(self, base, ic, oc, gain=1.0):
        self.tok(self.name(base), ic, oc)
        w = self.rng.normal(0.0, gain / np.sqrt(ic), size=(ic, oc)).astype(np.float32)
        self.floats(w)
        return w

    def matbias(self, base, c):
        self.tok(self.name(base), c)
        b = self.rng.normal(0.0, 0.1, c).astype(np.float32)
        self.floats(b)
        return b

    def tf_rmsnorm(self, base, c):
        self.tok(self.name(base), c, 1e-6)
        w = self.rng.uniform(0.9, 1.1, c).astype(np.float32)
        self.floats(w)
        return {"w": w, "eps": np.float32(1e-6)}


def _count_adds(blocks) -> int:
    return len(blocks)


def _write_block(w: _Writer, arch: Arch, spec, c: int, gain: float) -> dict:
    """Writes one block; returns its weights as a dict (the tree that write_model_tree returns)."""
    kind = spec[0]
    a = arch.act
    t = {"kind": kind}
    if kind == "res":
        cm = spec[1]
        w.tok("ordinary_block", w.name("res"))
        t["pre_bn"] = w.bn("bn", c); t["pre_act"] = w.act("act", a)
        t["regular"] = w.conv("conv", 3, c, cm)
        t["mid_bn"] = w.bn("bn", cm, gain=arch.mid_bn_gain); t["mid_act"] = w.act("act", a)
        t["final"] = w.conv("conv", 3, cm, c, gain=gain)
    elif kind == "gpool":
        cr, cg = spec[1], spec[2]
        w.tok("gpool_block", w.name("gpool"))
        t["pre_bn"] = w.bn("bn", c); t["pre_act"] = w.act("act", a)
        t["regular"] = w.conv("conv", 3, c, cr)
        t["gconv"] = w.conv("gconv", 3, c, cg)
        t["gbn"] = w.bn("gbn", cg); t["gact"] = w.act("gact", a)
        t["gmul"] = w.matmul("gmul", 3 * cg, cr)
        t["mid_bn"] = w.bn("bn", cr); t["mid_act"] = w.act("act", a)
        t["final"] = w.conv("conv", 3, cr, c, gain=gain)
    elif kind == "nbt":
        ci, inner = spec[1], spec[2]
        w.tok("nested_bottleneck_block", w.name("nbt"), len(inner))
        t["pre_bn"] = w.bn("bn", c); t["pre_act"] = w.act("act", a)
        t["regular"] = w.conv("preconv", 1, c, ci)
        g_in = 1.0 / np.sqrt(_count_adds(inner))
        t["inner"] = [_write_block(w, arch, b, ci, g_in) for b in inner]
        t["mid_bn"] = w.bn("bn", ci); t["mid_act"] = w.act("act", a)
        t["final"] = w.conv("postconv", 1, ci, c, gain=gain)
    elif kind == "attn":
        h, kvh, dq, dv, rope = spec[1:]
        w.tok("transformer_attention_block", w.name("attn"), h, kvh, dq, dv,
              int(rope != "none"), int(rope == "learnable"))
        t.update(heads=h, kv_heads=kvh, dq=dq, dv=dv, rope=rope)
        t["ln"] = w.tf_rmsnorm("ln", c)
        t["q"] = w.matmul("q", c, h * dq, gain=arch.qk_gain)
        t["k"] = w.matmul("k", c, kvh * dq, gain=arch.qk_gain)
        t["v"] = w.matmul("v", c, kvh * dv)
        t["o"] = w.matmul("o", h * dv, c, gain=gain)
        if rope == "learnable":
            w.tok(w.name("ropefreq"), kvh, dq // 2, 2)
            f = w.rng.uniform(-0.8, 0.8, size=(kvh, dq // 2, 2)).astype(np.float32)
            w.floats(f)
            t["freqs"] = f
        elif rope == "fixed":
            w.tok(w.name("ropetheta"), float(arch.rope_theta))
            t["theta"] = np.float32(arch.rope_theta)
    elif kind == "ffn":
        f, swiglu = spec[1], spec[2]
        w.tok("transformer_ffn_block", w.name("ffn"), c, f, int(bool(swiglu)))
        t["swiglu"] = bool(swiglu)
        t["ln"] = w.tf_rmsnorm("ln", c)
        t["l1"] = w.matmul("l1", c, f)
        if swiglu:
            t["lg"] = w.matmul("lg", c, f)
        t["l2"] = w.matmul("l2", f, c, gain=gain)
    else:
        raise ValueError(kind)
    return t


def write_model_tree(arch: Arch, seed: int, text_floats: bool = False):
    """The network `arch` with seeded weights: (bytes of a KataGo model file, weight tree). The floats are
    binary blocks, or text tokens (KataGo's .txt format) with `text_floats`."""
    rng = np.random.default_rng(seed)
    w = _Writer(rng, arch.model_version, text_floats)
    v = arch.model_version
    c = arch.trunk_c
    t = {"version": v, "P": num_policy_channels(arch), "S": num_score_channels(arch), "tip": arch.tip}
    w.tok(arch.name, v, arch.num_input_channels, arch.num_global_channels)
    if v >= 13:
        w.tok(20.0, 20.0, 20.0, 20.0, 40.0, 0.25, 30.0)
    if v >= 15:
        w.tok(arch.meta_encoder, 0, 0, 0, 0, 0, 0, 0)
    # Trunk header.
    w.tok("trunk", len(arch.blocks), c, arch.mid_c or c, arch.mid_c or c, 0, arch.gpool_c)
    if v >= 15:
        w.tok(1 if arch.tip.startswith("rms") else 0, 0, 0, 0, 0, 0)
    t["stem"] = w.conv("stem", arch.stem_k, arch.num_input_channels, c)
    t["stem_mm"] = w.matmul("stemglobal", arch.num_global_channels, c)
    if arch.meta_encoder:
        w.tok(w.name("metaenc"), 192)
        t["meta"] = {"m1": w.matmul("m1", 192, arch.meta_c), "b1": w.matbias("mb1", arch.meta_c),
                     "a1": w.act("ma1", arch.act)}
        t["meta"].update(m2=w.matmul("m2", arch.meta_c, arch.meta_c), b2=w.matbias("mb2", arch.meta_c),
                         a2=w.act("ma2", arch.act))
        t["meta"]["m3"] = w.matmul("m3", arch.meta_c, c)
    gain = 1.0 / np.sqrt(_count_adds(arch.blocks))
    t["blocks"] = [_write_block(w, arch, b, c, gain) for b in arch.blocks]
    if arch.tip == "bn":
        t["tip_bn"] = w.bn("tipbn", c)
    else:
        w.tok(w.name("tiprms"), c, 1e-5, int(arch.tip == "rms_spatial"), 0)
        gamma = rng.uniform(0.9, 1.1, c).astype(np.float32)
        beta = rng.normal(0.0, 0.1, c).astype(np.float32)
        w.floats(gamma)
        w.floats(beta)
        t["tip_rms"] = {"gamma": gamma, "beta": beta, "eps": np.float32(1e-5), "spatial": arch.tip == "rms_spatial"}
    t["tip_act"] = w.act("tipact", arch.act)
    # Policy head.
    p = num_policy_channels(arch)
    w.tok("policyhead")
    if v >= 17:
        w.tok(p, 0, 0, 0)
    h = {}
    h["p1"] = w.conv("p1", 1, c, arch.p1_c)
    h["g1"] = w.conv("g1", 1, c, arch.g1_c)
    h["g1_bn"] = w.bn("g1bn", arch.g1_c); h["g1_act"] = w.act("g1act", arch.act)
    h["gpool_bias"] = w.matmul("gpoolbias", 3 * arch.g1_c, arch.p1_c)
    h["p1_bn"] = w.bn("p1bn", arch.p1_c); h["p1_act"] = w.act("p1act", arch.act)
    h["p2"] = w.conv("p2", 1, arch.p1_c, p)
    if v >= 15:
        h["pass1"] = w.matmul("pass1", 3 * arch.g1_c, arch.p1_c)
        h["pass_b"] = w.matbias("passb", arch.p1_c)
        h["pass_act"] = w.act("passact", arch.act)
        h["pass2"] = w.matmul("pass2", arch.p1_c, p)
    else:
        h["pass1"] = w.matmul("pass", 3 * arch.g1_c, p)
    # Value head.
    s = num_score_channels(arch)
    w.tok("valuehead")
    if v >= 17:
        w.tok(0, 0, 0)
    h["v1"] = w.conv("v1", 1, c, arch.v1_c)
    h["v1_bn"] = w.bn("v1bn", arch.v1_c); h["v1_act"] = w.act("v1act", arch.act)
    h["v2"] = w.matmul("v2", 3 * arch.v1_c, arch.v2_c); h["v2_b"] = w.matbias("v2b", arch.v2_c)
    h["v2_act"] = w.act("v2act", arch.act)
    h["v3"] = w.matmul("v3", arch.v2_c, 3); h["v3_b"] = w.matbias("v3b", 3)
    h["sv3"] = w.matmul("sv3", arch.v2_c, s); h["sv3_b"] = w.matbias("sv3b", s)
    h["own"] = w.conv("own", 1, arch.v1_c, 1)
    t["heads"] = h
    return w.buf.getvalue(), t


def write_model(arch: Arch, seed: int) -> bytes:
    """The network `arch` with seeded weights, as the bytes of a KataGo binary model file."""
    return write_model_tree(arch, seed)[0]


# ---------------------------------------------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------------------------------------------

def make_inputs(n: int, seed: int, board_sizes: Optional[List[int]] = None, num_input_channels: int = 22,
                num_global: int = 19, meta: int = 0):
    """Seeded inputs as the benchmark draws them: spatial [n, C, 19, 19] with plane 0 the on-board mask and
    the other planes Bernoulli(0.3) on board (0 off board), global [n, G] with rule flags in {0, 1} and the
    komi slot (5) in U(-1, 1), and meta [n, 192] rows in U(0, 1) when `meta`. `board_sizes` gives each row's
    board side (default 19: full board)."""
    rng = np.random.default_rng(seed)
    spatial = (rng.random((n, num_input_channels, POS_LEN, POS_LEN)) < 0.3).astype(np.float32)
    for i in range(n):
        bs = POS_LEN if board_sizes is None else board_sizes[i % len(board_sizes)]
        m = np.zeros((POS_LEN, POS_LEN), np.float32)
        m[:bs, :bs] = 1.0
        spatial[i] *= m[None]
        spatial[i, 0] = m
    glob = (rng.random((n, num_global)) < 0.5).astype(np.float32)
    if num_global > 5:
        glob[:, 5] = rng.uniform(-1.0, 1.0, n).astype(np.float32)
    meta_rows = rng.random((n, 192)).astype(np.float32) if meta else None
    return spatial, glob, meta_rows


def make_positions(n: int, seed: int, size: int = 19):
    """Seeded positions for the device featurizer (fields of kg_position, as dicts for make_positions): boards of
    `size` x `size` with stones on about half the points (Bernoulli(0.5), each colour alike), area rules with a
    komi of 7.5 from white's side, a few ko, superko and ladder marks, and five alternating history moves."""
    rng = np.random.default_rng(seed)
    out = []
    npts = size * size
    for _ in range(n):
        pla = int(rng.integers(1, 3))
        color = np.zeros(361, np.uint8)
        color[:npts] = np.where(rng.random(npts) < 0.5, rng.integers(1, 3, npts), 0)
        marks = np.zeros(361, np.uint8)
        marks[:npts] = (rng.random(npts) < 0.05) * rng.integers(1, 64, npts)
        area = np.zeros(361, np.uint8)
        area[:npts] = color[:npts]
        empties = np.flatnonzero(color[:npts] == 0)
        moves = np.zeros(10, np.int32)
        for k in range(5):
            moves[2 * k] = int(rng.integers(0, npts))
            moves[2 * k + 1] = 3 - pla if k % 2 == 0 else pla
        meta = np.array([size, size, pla, int(empties[0]) if len(empties) else -1, 0, 0, 0, 0, 0, 0, 0, 5, 5],
                        np.int32)
        out.append(dict(meta=meta, color=color, marks=marks, area=area, enc=np.zeros(361, np.uint8), moves=moves,
                        self_komi=7.5 if pla == 2 else -7.5, pda=0.0))
    return out
