"""An independent float64 reference of the forward pass, composed from torch's CPU library routines
(conv2d, matmul, softplus, softmax) over the weight tree of katago-rs_amd.synth.write_model_tree.

It follows the op graph of tools/bin2onnx/bin2onnx.py (GraphBuilder, :1088-1531) node by node, including its
RoPE formulation on permuted projection columns (:1345-1374) where the oracle rotates interleaved pairs; it is
used to pin the CPU oracle, not the product.
"""

import numpy as np
import torch
import torch.nn.functional as F

HW = 361
D = torch.float64


def _t(a):
    return torch.as_tensor(np.asarray(a, np.float64))


def bn_merged(bn):
    """computeMerged in float32 (bin2onnx.py:179-184)."""
    s = (bn["gamma"] / np.sqrt(bn["var"] + np.float32(bn["eps"]))).astype(np.float32)
    b = (bn["beta"] - s * bn["mean"]).astype(np.float32)
    return _t(s), _t(b)


def act(x, kind):
    if kind == "ACTIVATION_RELU":
        return torch.relu(x)
    if kind == "ACTIVATION_MISH":
        return x * torch.tanh(F.softplus(x, beta=1.0, threshold=20.0))
    if kind == "ACTIVATION_SILU":
        return x / (torch.exp(-x) + 1.0)
    return x


class Ref:
    def __init__(self, tree):
        self.t = tree

    def conv(self, x, w):
        k = w.shape[-1]
        return F.conv2d(x, _t(w), padding=k // 2)

    def bn_act_mask(self, x, bn, a):
        s, b = bn_merged(bn)
        return act(x * s[None, :, None, None] + b[None, :, None, None], a) * self.mask

    def gpool(self, x):
        n, c = x.shape[:2]
        flat = x.reshape(n, c, HW)
        mean = flat.sum(2) / self.mask_sum
        mx = (flat + self.max_bias).amax(2)
        return torch.cat([mean, mean * self.s1, mx], 1)

    def value_pool(self, x):
        n, c = x.shape[:2]
        mean = x.reshape(n, c, HW).sum(2) / self.mask_sum
        return torch.cat([mean, mean * self.s1, mean * self.s2], 1)

    # --- transformer (tokens [N, S, C]) ---
    def rmsnorm_tok(self, x, ln):
        ms = (x * x).sum(2, keepdim=True) / x.shape[2]
        rms = 1.0 / torch.sqrt(ms + float(ln["eps"]))
        return x * rms * _t(ln["w"]) * self.mask_tok

    @staticmethod
    def rope_tables(b):
        """computeRopeCosSin (bin2onnx.py:449-485): float32 angles, cos/sin through float64."""
        f32 = np.float32
        dq = b["dq"]
        pairs = dq // 2
        ys, xs = np.meshgrid(np.arange(19), np.arange(19), indexing="ij")
        xf = xs.reshape(-1).astype(f32)
        yf = ys.reshape(-1).astype(f32)
        if b["rope"] == "learnable":
            fr = b["freqs"]
            ang = (xf[None, None, :] * fr[:, :, 0:1]).astype(f32) + (yf[None, None, :] * fr[:, :, 1:2]).astype(f32)
            ang = ang.astype(np.float64)
            return np.cos(ang).astype(f32), np.sin(ang).astype(f32)
        per = pairs // 2
        cos = np.zeros((pairs, HW), f32)
        sin = np.zeros_like(cos)
        for p in range(pairs):
            padj = p if p < per else p - per
            expo = f32(f32(2 * padj) / f32(pairs))
            powv = f32(np.power(np.float64(f32(b["theta"])), np.float64(expo)))
            freq = f32(f32(1.0) / powv)
            pos = yf if p < per else xf
            a = (pos * freq).astype(f32).astype(np.float64)
            cos[p], sin[p] = np.cos(a).astype(f32), np.sin(a).astype(f32)
        return cos, sin

    def attention(self, x, b):
        n = x.shape[0]
        nh, nkv, hd, vhd = b["heads"], b["kv_heads"], b["dq"], b["dv"]
        g = nh // nkv
        xn = self.rmsnorm_tok(x, b["ln"])
        wq, wk = b["q"], b["k"]
        rope = b["rope"] != "none"
        half = hd // 2
        if rope:
            perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])
            wq = wq[:, (np.arange(nh)[:, None] * hd + perm[None, :]).reshape(-1)]
            wk = wk[:, (np.arange(nkv)[:, None] * hd + perm[None, :]).reshape(-1)]
        q = torch.matmul(xn, _t(wq)).reshape(n, HW, nh, hd).permute(0, 2, 1, 3)
        k = torch.matmul(xn, _t(wk)).reshape(n, HW, nkv, hd).permute(0, 2, 1, 3)
        v = torch.matmul(xn, _t(b["v"])).reshape(n, HW, nkv, vhd).permute(0, 2, 1, 3)
        if rope:
            cos, sin = self.rope_tables(b)
            if b["rope"] == "learnable":
                ck = _t(cos.transpose(0, 2, 1))[None]  # [1, nkv, S, P]
                sk = _t(sin.transpose(0, 2, 1))[None]
                kv_of = np.arange(nh) * nkv // nh
                cq, sq = ck[:, kv_of], sk[:, kv_of]
            else:
                ck = cq = _t(cos.T)[None, None]
                sk = sq = _t(sin.T)[None, None]

            def rot(z, c, s):
                z0, z1 = z[..., :half], z[..., half:]
                return torch.cat([z0 * c - z1 * s, z0 * s + z1 * c], -1)

            q = rot(q, cq, sq)
            k = rot(k, ck, sk)
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        scores = torch.matmul(q, k.transpose(2, 3)) * scale + self.attn_bias
        o = torch.matmul(torch.softmax(scores, dim=3), v)
        o = o.permute(0, 2, 1, 3).reshape(n, HW, nh * vhd)
        return x + torch.matmul(o, _t(b["o"])) * self.mask_tok

    def ffn(self, x, b):
        xn = self.rmsnorm_tok(x, b["ln"])
        a = torch.matmul(xn, _t(b["l1"]))
        if b["swiglu"]:
            h = act(a, "ACTIVATION_SILU") * torch.matmul(xn, _t(b["lg"]))
        else:
            h = act(a, "ACTIVATION_MISH")
        return x + torch.matmul(h, _t(b["l2"])) * self.mask_tok

    def stack(self, x, blocks):
        for b in blocks:
            k = b["kind"]
            c = x.shape[1]
            if k in ("attn", "ffn"):
                n = x.shape[0]
                tok = x.reshape(n, c, HW).transpose(1, 2)
                tok = self.attention(tok, b) if k == "attn" else self.ffn(tok, b)
                x = tok.transpose(1, 2).reshape(n, c, 19, 19)
            elif k == "res":
                t = self.conv(self.bn_act_mask(x, b["pre_bn"], b["pre_act"]), b["regular"])
                t = self.conv(self.bn_act_mask(t, b["mid_bn"], b["mid_act"]), b["final"])
                x = x + t
            elif k == "gpool":
                t = self.bn_act_mask(x, b["pre_bn"], b["pre_act"])
                reg = self.conv(t, b["regular"])
                g = self.bn_act_mask(self.conv(t, b["gconv"]), b["gbn"], b["gact"])
                bias = torch.matmul(self.gpool(g), _t(b["gmul"]))
                reg = reg + bias[:, :, None, None]
                x = x + self.conv(self.bn_act_mask(reg, b["mid_bn"], b["mid_act"]), b["final"])
            elif k == "nbt":
                t = self.conv(self.bn_act_mask(x, b["pre_bn"], b["pre_act"]), b["regular"])
                t = self.stack(t, b["inner"])
                x = x + self.conv(self.bn_act_mask(t, b["mid_bn"], b["mid_act"]), b["final"])
        return x

    def forward(self, spatial, glob, meta=None):
        t = self.t
        n = spatial.shape[0]
        x = _t(spatial)
        self.mask = x[:, 0:1]
        mflat = self.mask.reshape(n, 1, HW)
        self.mask_sum = mflat.sum(2)
        c = torch.sqrt(self.mask_sum) - 14.0
        self.s1 = c * 0.1
        self.s2 = c * c * 0.01 - 0.1
        self.max_bias = mflat * 1e4 - 1e4
        self.mask_tok = self.mask.reshape(n, HW, 1)
        self.attn_bias = self.mask.reshape(n, 1, 1, HW) * 3e4 - 3e4
        h = self.conv(x, t["stem"]) + torch.matmul(_t(glob), _t(t["stem_mm"]))[:, :, None, None]
        if "meta" in t:
            m = t["meta"]
            z = act(torch.matmul(_t(meta), _t(m["m1"])) + _t(m["b1"]), m["a1"])
            z = act(torch.matmul(z, _t(m["m2"])) + _t(m["b2"]), m["a2"])
            h = h + torch.matmul(z, _t(m["m3"]))[:, :, None, None]
        h = self.stack(h, t["blocks"])
        if "tip_bn" in t:
            tip = self.bn_act_mask(h, t["tip_bn"], t["tip_act"])
        else:
            r = t["tip_rms"]
            C = h.shape[1]
            if r["spatial"]:
                ss = (h * h * self.mask).reshape(n, -1).sum(1) / (self.mask_sum[:, 0] * C)
                rms = (1.0 / torch.sqrt(ss + float(r["eps"])))[:, None, None, None]
            else:
                rms = 1.0 / torch.sqrt((h * h).sum(1, keepdim=True) / C + float(r["eps"]))
            y = h * rms * _t(r["gamma"])[None, :, None, None] + _t(r["beta"])[None, :, None, None]
            tip = act(y, t["tip_act"]) * self.mask
        hd = t["heads"]
        p1 = self.conv(tip, hd["p1"])
        g1 = self.bn_act_mask(self.conv(tip, hd["g1"]), hd["g1_bn"], hd["g1_act"])
        g1p = self.gpool(g1)
        p1 = p1 + torch.matmul(g1p, _t(hd["gpool_bias"]))[:, :, None, None]
        p1 = self.bn_act_mask(p1, hd["p1_bn"], hd["p1_act"])
        p2 = self.conv(p1, hd["p2"]).reshape(n, t["P"], HW)
        if t["version"] >= 15:
            pas = act(torch.matmul(g1p, _t(hd["pass1"])) + _t(hd["pass_b"]), hd["pass_act"])
            pas = torch.matmul(pas, _t(hd["pass2"]))
        else:
            pas = torch.matmul(g1p, _t(hd["pass1"]))
        policy = torch.cat([p2, pas[:, :, None]], 2)
        v1 = self.bn_act_mask(self.conv(tip, hd["v1"]), hd["v1_bn"], hd["v1_act"])
        v2 = act(torch.matmul(self.value_pool(v1), _t(hd["v2"])) + _t(hd["v2_b"]), hd["v2_act"])
        value = torch.matmul(v2, _t(hd["v3"])) + _t(hd["v3_b"])
        score = torch.matmul(v2, _t(hd["sv3"])) + _t(hd["sv3_b"])
        own = self.conv(v1, hd["own"]).reshape(n, HW)
        return torch.cat([policy.reshape(n, -1), value, score, own], 1).numpy()
