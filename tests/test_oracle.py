"""Pins the CPU oracle (CPU-only tests).

The oracle restates the reference's forward pass; these tests check it against what the mathematics and
independent library routines fix: the Winograd F(4x4,3x3) identity, torch's float64 conv2d, an independent
float64 forward built from torch library ops over the same weights (tests/torch_ref.py, which follows
bin2onnx's graph node by node), the dihedral symmetry group, and the reference's bucket cases.
"""

import gzip
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import torch_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_winograd_restatement_equals_direct_convolution(oracle):
    rng = np.random.default_rng(7)
    for n, ic, oc in [(1, 3, 5), (2, 7, 4)]:
        x = rng.normal(size=(n, ic, 19, 19))
        w = rng.normal(size=(oc, ic, 3, 3))
        y_w = oracle.conv3x3_winograd(x, w)
        y_d = oracle.conv_direct(x, w)
        assert np.abs(y_w - y_d).max() <= 1e-12 * np.abs(y_d).max()


def test_winograd_filter_transform_against_lavin_gray_matrices(oracle):
    # F(4x4, 3x3) matrices as published (Lavin & Gray 2015): out = A^T [(G g G^T) * (B^T d B)] A is the 4x4
    # correlation of the 6x6 tile d with g.
    G = np.array([[1 / 4, 0, 0], [-1 / 6, -1 / 6, -1 / 6], [-1 / 6, 1 / 6, -1 / 6], [1 / 24, 1 / 12, 1 / 6],
                  [1 / 24, -1 / 12, 1 / 6], [0, 0, 1]])
    BT = np.array([[4, 0, -5, 0, 1, 0], [0, -4, -4, 1, 1, 0], [0, 4, -4, -1, 1, 0], [0, -2, -1, 2, 1, 0],
                   [0, 2, -1, -2, 1, 0], [0, 4, 0, -5, 0, 1]], float)
    AT = np.array([[1, 1, 1, 1, 1, 0], [0, 1, -1, 2, -2, 0], [0, 1, 1, 4, 4, 0], [0, 1, -1, 8, -8, 1]], float)
    rng = np.random.default_rng(3)
    g = rng.normal(size=(3, 3))
    d = rng.normal(size=(6, 6))
    direct = np.array([[np.sum(d[i:i + 3, j:j + 3] * g) for j in range(4)] for i in range(4)])
    assert np.allclose(AT @ ((G @ g @ G.T) * (BT @ d @ BT.T)) @ AT.T, direct, atol=1e-12)
    # The oracle's filter transform ([36][ic][oc], point p = 6*row + col) equals G g G^T.
    w = rng.normal(size=(2, 3, 3, 3))
    U = oracle.wino_filter(w)
    for o in range(2):
        for i in range(3):
            assert np.allclose(U[:, i, o].reshape(6, 6), G @ w[o, i] @ G.T, atol=1e-14)


@pytest.mark.parametrize("k", [1, 3, 5])
def test_direct_convolution_matches_torch(oracle, k):
    rng = np.random.default_rng(k)
    x = rng.normal(size=(2, 4, 19, 19))
    w = rng.normal(size=(3, 4, k, k))
    y = oracle.conv_direct(x, w)
    t = F.conv2d(torch.tensor(x), torch.tensor(w), padding=k // 2).numpy()
    assert np.abs(y - t).max() <= 1e-12 * np.abs(t).max()


def _tiny(synth):
    return synth.tiny_nets()


@pytest.mark.parametrize("name", ["t_res", "t_nbt", "t_v8", "t_tf", "t_tf64", "t_human", "t_rms", "t_rmspos"])
def test_oracle_matches_independent_torch_forward(oracle, synth, name):
    arch = _tiny(synth)[name]
    mb, tree = synth.write_model_tree(arch, 11)
    sp, gl, me = synth.make_inputs(3, 5, board_sizes=[19, 9, 13], meta=arch.meta_encoder)
    out = oracle.Model(mb).forward(sp, gl, me)
    ref = torch_ref.Ref(tree).forward(sp, gl, me)
    assert np.abs(out - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())


def test_oracle_reproduces_golden_fixtures(oracle, synth):
    g = np.load(os.path.join(GOLDEN, "oracle_tiny.npz"))
    m0 = np.load(os.path.join(GOLDEN, "m0_inputs.npz"))
    for name, arch in _tiny(synth).items():
        model = oracle.Model(synth.write_model(arch, 1))
        meta = g[f"{name}.meta"] if f"{name}.meta" in g else None
        out = model.forward(g[f"{name}.spatial"], g[f"{name}.glob"], meta)
        assert np.abs(out - g[f"{name}.out"]).max() <= 1e-12 * max(1.0, np.abs(out).max()), name
        out = model.forward(m0["spatial"], m0["glob"], m0["meta"] if arch.meta_encoder else None)
        assert np.abs(out - g[f"{name}.m0_out"]).max() <= 1e-12 * max(1.0, np.abs(out).max()), name


def test_oracle_float32_path_close_to_float64(oracle, synth):
    arch = _tiny(synth)["t_nbt"]
    model = oracle.Model(synth.write_model(arch, 2))
    sp, gl, _ = synth.make_inputs(2, 9)
    a = model.forward(sp, gl)
    b = model.forward(sp, gl, dtype=np.float32)
    assert np.abs(a - b).max() <= 1e-5 * np.abs(a).max()


def test_oracle_rows_are_independent(oracle, synth):
    arch = _tiny(synth)["t_tf"]
    model = oracle.Model(synth.write_model(arch, 4))
    sp, gl, _ = synth.make_inputs(3, 1, board_sizes=[19, 7, 13])
    both = model.forward(sp, gl)
    for i in range(3):
        one = model.forward(sp[i:i + 1], gl[i:i + 1])
        assert np.array_equal(one[0], both[i])


def test_full_board_pooling_constants(oracle, synth):
    # On a full 19x19 board area = 361, so (sqrt(area) - 14) * 0.1 = 0.5 and (sqrt - 14)^2 * 0.01 - 0.1 = 0.15
    # (bin2onnx.py:1203-1220): the value pool of a constant map c is [c, 0.5 c, 0.15 c].
    r = torch_ref.Ref({})
    n = 1
    mask = torch.ones(n, 1, 19, 19, dtype=torch.float64)
    r.mask = mask
    r.mask_sum = mask.reshape(n, 1, 361).sum(2)
    cc = torch.sqrt(r.mask_sum) - 14.0
    r.s1, r.s2 = cc * 0.1, cc * cc * 0.01 - 0.1
    x = torch.full((1, 2, 19, 19), 3.0, dtype=torch.float64)
    vp = r.value_pool(x).numpy()[0]
    assert np.allclose(vp, [3, 3, 1.5, 1.5, 0.45, 0.45], atol=1e-12)


def _dihedral(a, s):
    """The eight symmetries of a square array by the reference's bit meaning for outputs (reverse)."""
    out = a
    if s & 4:
        out = out.T
    if s & 1:
        out = out[::-1, :]
    if s & 2:
        out = out[:, ::-1]
    return out


def test_symmetry_group(oracle):
    rng = np.random.default_rng(0)
    src = rng.normal(size=(1, 2, 19, 19)).astype(np.float32)
    imgs = []
    for s in range(8):
        fwd = oracle.copy_with_symmetry(src, s)
        back = oracle.copy_with_symmetry(fwd, s, reverse=True)
        assert np.array_equal(back, src), s  # outputs map back through the same symmetry
        rev = oracle.copy_with_symmetry(src, s, reverse=True)
        assert np.array_equal(rev[0, 0], np.ascontiguousarray(_dihedral(src[0, 0], s))), s
        imgs.append(fwd[0, 0].tobytes())
    assert len(set(imgs)) == 8
    # Bit meanings on inputs: 1 flips rows (y), 2 flips columns (x), 4 transposes.
    p = src[0, 0]
    assert np.array_equal(oracle.copy_with_symmetry(src, 1)[0, 0], p[::-1, :])
    assert np.array_equal(oracle.copy_with_symmetry(src, 2)[0, 0], p[:, ::-1])
    assert np.array_equal(oracle.copy_with_symmetry(src, 4)[0, 0], p.T)
    # NHWC and NCHW agree.
    nhwc = oracle.copy_with_symmetry(np.ascontiguousarray(src.transpose(0, 2, 3, 1)), 6, nhwc=True)
    assert np.array_equal(nhwc.transpose(0, 3, 1, 2), oracle.copy_with_symmetry(src, 6))


def test_padded_batch_size_reference_cases(oracle):
    # crates/katago-nn-burn/tests/batch_buckets.rs:27-35
    b = [1, 2, 4, 8, 16, 32]
    assert oracle.padded_batch_size(b, 1, 32) == 1
    assert oracle.padded_batch_size(b, 3, 32) == 4
    assert oracle.padded_batch_size(b, 17, 32) == 32
    assert oracle.padded_batch_size(b, 17, 24) == 17
    assert oracle.padded_batch_size([], 5, 32) == 5


def test_model_file_variants_parse_alike(oracle, synth):
    arch = _tiny(synth)["t_human"]
    mb, _ = synth.write_model_tree(arch, 3)
    txt, _ = synth.write_model_tree(arch, 3, text_floats=True)
    sp, gl, me = synth.make_inputs(2, 1, meta=1)
    a = oracle.Model(mb).forward(sp, gl, me)
    assert np.array_equal(a, oracle.Model(txt).forward(sp, gl, me))
    assert np.array_equal(a, oracle.Model(gzip.compress(mb)).forward(sp, gl, me))


def test_operand_rounding_matches_float16_and_bfloat16(oracle):
    """The 16-bit operand emulation rounds like numpy's float16 and like a float32 -> bfloat16 conversion."""
    import torch
    rng = np.random.default_rng(0)
    x = rng.normal(size=100000) * np.exp(rng.uniform(-20, 12, 100000))
    x[:5] = [0.0, -0.0, 65504.0, 65520.0, 2.0 ** -25]  # max, overflow to inf, half the smallest subnormal
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float64)
    got = oracle.round_operands(x, "f16")
    assert np.array_equal(got, want)
    # bfloat16 from float32 values (the device rounds float32): exact.
    x32 = x.astype(np.float32).astype(np.float64)
    want_bf = torch.tensor(x32, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    assert np.array_equal(oracle.round_operands(x32, "bf16"), want_bf)


def test_operand_emulation_without_rounding_is_the_float64_forward(oracle, synth):
    mb = synth.write_model(synth.tiny_nets()["t_nbt"], 1)
    sp, gl, _ = synth.make_inputs(2, 3)
    m = oracle.Model(mb)
    ref = m.forward(sp, gl)
    assert np.array_equal(m.forward(sp, gl, operands="f16", acts=False, weights=False), ref)
    q = m.forward(sp, gl, operands="f16")
    assert 0 < np.abs(q - ref).max() < 2e-2


def test_oracle_copy_outputs_sentinels_follow_every_reference_branch(oracle):
    """The oracle's copy_outputs restatement on sentinel rows, against the branch-by-branch reading of
    backend.rs:622-731 (tests/outputs_spec.py) and the brute-force-pinned symmetry copy."""
    import outputs_spec as spec
    for v, P in spec.CASES:
        S = spec.score_channels(v)
        raw = spec.sentinel_row(P, S)
        for opt in spec.OPTIMISMS:
            pol, fields, own = spec.expected(raw, P, S, v, opt)
            for sym in (0, 6):
                gp, gf, go = oracle.copy_outputs_row(raw, P, S, v, sym, opt)
                wp = np.append(oracle.copy_with_symmetry(pol[:361].reshape(1, 1, 19, 19), sym, reverse=True).ravel(),
                               pol[361])
                assert np.array_equal(gp, wp), (v, P, opt, sym)
                assert np.array_equal(gf, fields), (v, P, opt, sym, gf, fields)
                assert np.array_equal(go, oracle.copy_with_symmetry(own.reshape(1, 1, 19, 19), sym,
                                                                    reverse=True).ravel()), (v, P, opt, sym)


def _post_row(P, S, rng):
    row = rng.normal(0.0, 1.0, size=P * 362 + 3 + S + 361).astype(np.float32)
    return row


def test_oracle_postprocess_policy_closed_forms(oracle):
    """NNEvaluator's policy softmax (nneval.rs:1223-1292) against closed forms: two legal moves give the logistic
    of their scaled difference; illegal moves are -1; the passing cap gives a dominant pass exactly 19 / 20; the
    legal probabilities sum to 1."""
    rng = np.random.default_rng(1)
    row = _post_row(1, 6, rng)
    legal = np.zeros(362, np.uint8)
    legal[[10, 200]] = 1
    for temp in (1.0, 0.5, 2.0):
        st, pol, _, _ = oracle.postprocess_row(row, 1, 6, 14, 0, 0.0, legal, True, 19, 19, temp)
        a, b = float(row[10]) / np.float32(temp), float(row[200]) / np.float32(temp)
        assert st == 0
        assert abs(pol[10] - 1.0 / (1.0 + np.exp(b - a))) < 1e-6
        assert abs(pol[10] + pol[200] - 1.0) < 1e-6
        assert np.all(np.delete(pol, [10, 200]) == -1.0)
    legal = np.ones(362, np.uint8)
    row2 = row.copy()
    row2[361] = 20.0  # dominant, yet the others sum (times 19) stays above the 1e-20 floor
    st, pol, _, _ = oracle.postprocess_row(row2, 1, 6, 14, 0, 0.0, legal, True, 19, 19, 1.0, True)
    assert st == 0 and abs(pol[361] - 0.95) < 1e-6 and abs(pol.sum() - 1.0) < 1e-5
    st, pol, _, _ = oracle.postprocess_row(row2, 1, 6, 14, 0, 0.0, legal, True, 19, 19, 1.0, False)
    assert pol[361] > 0.9999  # without the cap the pass takes nearly everything


def test_oracle_postprocess_value_closed_forms(oracle):
    """The value and score transforms (nneval.rs:1298-1477) against closed forms: the value softmax sums to 1 and
    swaps win and loss for black to move; no-result is 0 when the rules exclude it; version 9 score mean is
    raw * 20 * (1 - noresult) and the stdev a softplus; version 3's score is 2 sqrt(area) times the raw value
    (tan of its own arctan); ownership is +-tanh of the symmetry-mapped raw value and 0 off the board."""
    rng = np.random.default_rng(2)
    row = _post_row(1, 6, rng)
    legal = np.ones(362, np.uint8)
    st, _, fw, own_w = oracle.postprocess_row(row, 1, 6, 9, 0, 0.0, legal, True, 13, 13)
    st2, _, fb, own_b = oracle.postprocess_row(row, 1, 6, 9, 0, 0.0, legal, False, 13, 13)
    assert st == 0 and st2 == 0
    v = row[362:365].astype(np.float64)
    e = np.exp(v - v.max())
    e /= e.sum()
    assert np.allclose(fw[:3], e, rtol=1e-6) and np.allclose(fb[:3], [e[1], e[0], e[2]], rtol=1e-6)
    s = row[365:371].astype(np.float64)
    mean = s[0] * 20.0 * (1.0 - e[2])
    stdev = np.log1p(np.exp(s[1])) * 20.0
    assert abs(fw[3] - mean) <= 1e-5 * max(1.0, abs(mean)) and abs(fb[3] + mean) <= 1e-5 * max(1.0, abs(mean))
    assert abs(fw[4] - (s[0] * 20.0) ** 2 * (1.0 - e[2]) - stdev ** 2 * (1.0 - e[2])) <= 1e-4 * max(1.0, fw[4])
    own_raw = row[371:].reshape(19, 19)
    expect = np.tanh(own_raw.astype(np.float64))
    expect[13:, :] = 0.0
    expect[:, 13:] = 0.0
    assert np.allclose(own_w.reshape(19, 19), expect, atol=1e-6) and np.allclose(own_b, -own_w)
    st, _, fr, _ = oracle.postprocess_row(row, 1, 6, 9, 0, 0.0, legal, True, 19, 19, no_result_allowed=False)
    assert st == 0 and fr[2] == 0.0 and abs(fr[0] + fr[1] - 1.0) < 1e-6
    # Version 3: one score channel; tan(atan(x)) = x, times 2 sqrt(board area).
    row3 = _post_row(1, 1, rng)
    row3[365] = 0.3
    st, _, f3, _ = oracle.postprocess_row(row3, 1, 1, 3, 0, 0.0, legal, True, 9, 9)
    assert st == 0 and abs(f3[3] - 0.3 * 2.0 * 9.0) < 1e-5 and f3[4] == np.float32(f3[3]) * np.float32(f3[3])
    assert f3[6] == -1.0 and f3[7] == -1.0 and f3[8] == -1.0
    # Nonfinite inputs: the reference's two errors.
    bad = row.copy()
    bad[:362] = np.inf
    assert oracle.postprocess_row(bad, 1, 6, 9, 0, 0.0, legal, True, 19, 19)[0] == 1
    bad = row.copy()
    bad[362] = np.inf
    assert oracle.postprocess_row(bad, 1, 6, 9, 0, 0.0, legal, True, 19, 19)[0] == 2


def _skipnn_rows():
    """The evaluations of tests/golden/nneval_skipnn.npz as raw rows (P = 2 equal policy channels, so the optimism
    mix leaves them unchanged; S = 6; symmetry 0) with their post-processing inputs."""
    z = np.load(os.path.join(GOLDEN, "nneval_skipnn.npz"))
    rows = np.zeros((len(z["line"]), 2 * 362 + 3 + 6 + 361), np.float32)
    rows[:, :362] = z["raw_policy"]
    rows[:, 362:724] = z["raw_policy"]
    rows[:, 724:727] = z["raw_value"]
    rows[:, 727:733] = z["raw_score"]
    rows[:, 733:] = z["raw_owner"]
    return z, rows


def test_skipnn_generator_known_answers():
    """The Rand restatement behind tests/golden/nneval_skipnn.npz: the known-answer sequences of the reference's
    own generator self-tests (core/rand.rs XorShift1024Mult::test, PCG32::test)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("gen_nneval_skipnn", os.path.join(GOLDEN, "gen_nneval_skipnn.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    gen.check_generators()


def test_oracle_postprocess_matches_reference_skipnn_fixture(oracle):
    """NNEvaluator's post-processing (nneval.rs:1197-1500, model version 17, default post-process parameters) of
    the reference's own skip-NN evaluations (fixtures/upstream-v1.18.2/unit/oracle/nneval_skipnn.txt, regenerated
    by tests/golden/gen_nneval_skipnn.py): 19 evaluations on boards from 6x6 to 19x19, with and without the
    passing hack and owner map, both players to move, rules with and without no-result. Every policy probability,
    value field and ownership value equals the fixture's float bits."""
    z, rows = _skipnn_rows()
    for i in range(len(rows)):
        bx, by = (int(v) for v in z["board"][i])
        st, pol, fields, own = oracle.postprocess_row(
            rows[i], 2, 6, 17, 0, float(np.float32(z["optimism"][i])), z["legal"][i], bool(z["white"][i]), bx, by,
            float(z["temperature"][i]), bool(z["passing"][i]), bool(z["no_result"][i]))
        what = f"fixture line {int(z['line'][i])}"
        assert st == 0, what
        assert np.array_equal(pol.view(np.uint32), z["exp_policy"][i]), what
        assert np.array_equal(fields.view(np.uint32), z["exp_fields"][i]), what
        if z["owner"][i]:
            assert np.array_equal(own.view(np.uint32), z["exp_owner"][i]), what
