"""The device output post-processing (kg_post_outputs, kg_get_output_eval): copy_outputs
(crates/katago-nn-burn/src/backend.rs:622-731) and NNEvaluator's arithmetic on the fields
(crates/katago-core/src/neuralnet/nneval.rs:1197-1500), against the oracle's restatement
(oracle.postprocess_row), on the device through the C ABI.

Bit for bit: the device computes the policy softmax as the reference does (glibc's expf, the maximum from -1e25,
the sum in position order), ownership as the correctly rounded tanhf, and the value and score fields in double with
one rounding to float, so every policy probability, ownership value and field equals the oracle's (which the
reference's own skip-NN fixture pins bit for bit), except the model-version-3 score path through atanf and tan
(the device's own, 1e-5 relative). Illegal moves are -1 and off-board ownership 0.
"""

import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

VERSIONS = {  # model version -> (spatial, global) input channels of that version
    3: (22, 14), 5: (22, 14), 8: (22, 19), 9: (22, 19), 10: (22, 19), 14: (22, 19), 16: (22, 19), 17: (22, 19),
}


def _arch(synth, v):
    base = synth.tiny_nets()["t_v8"]
    sp, gl = VERSIONS[v]
    extra = {"policy_channels": 2} if v >= 17 else {}
    return dataclasses.replace(base, model_version=v, num_input_channels=sp, num_global_channels=gl,
                               name=f"t-post-v{v}", **extra)


def _cases(rng, n, row_len):
    raw = np.empty((n, row_len), np.float32)
    raw[:] = rng.normal(0.0, 1.0, size=raw.shape)
    raw[:, :362 * 4] *= 2.0
    post, sym, opt = [], rng.integers(0, 8, n), rng.uniform(0.0, 1.0, n).astype(np.float32)
    for i in range(n):
        bx, by = [(19, 19), (13, 13), (9, 9), (19, 13), (7, 11)][i % 5]
        legal = (rng.uniform(size=362) < 0.7).astype(np.uint8)
        off = np.array([(p // 19 >= by or p % 19 >= bx) for p in range(361)] + [False])
        legal[off] = 0
        legal[361] = 1
        post.append({"legal": legal, "white_to_move": bool(i % 2), "board_x_size": bx, "board_y_size": by,
                     "nn_policy_temperature": [1.0, 0.5, 1.3][i % 3], "enable_passing_hacks": bool(i % 4 == 1),
                     "no_result_allowed": bool(i % 3 != 2)})
    return raw, sym, opt, post


def _compare(res, ref, v, what):
    st, pol, fields, own = ref
    assert st == 0, f"{what}: oracle status {st}"
    bits = lambda x: np.asarray(x, np.float32).view(np.uint32)
    p = res["policy"]
    nd = int(np.count_nonzero(bits(p) != bits(pol)))
    assert nd == 0, f"{what}: {nd} policy values differ (max {np.abs(p - pol).max():.3e})"
    names = ["white_win_prob", "white_loss_prob", "white_no_result_prob", "white_score_mean", "white_score_mean_sq",
             "white_lead", "var_time_left", "shortterm_winloss_error", "shortterm_score_error"]
    for k, name in enumerate(names):
        a, b = np.float32(res[name]), np.float32(fields[k])
        if v == 3 and k in (3, 4, 5):  # the score path through atanf and tan
            assert abs(float(a) - float(b)) <= 1e-5 * max(1.0, abs(float(b))), f"{what}: {name} {a} vs {b}"
        else:
            assert bits(a) == bits(b), f"{what}: {name} {a!r} vs {b!r}"
    no = int(np.count_nonzero(bits(res["ownership"]) != bits(own)))
    assert no == 0, f"{what}: {no} ownership values differ (max {np.abs(res['ownership'] - own).max():.3e})"


@pytest.mark.parametrize("v", sorted(VERSIONS))
def test_post_outputs_match_oracle(kgx, synth, oracle, v):
    arch = _arch(synth, v)
    net = kgx.Net(synth.write_model(arch, 3))
    h = kgx.Handle(net, 8, "f32")
    rng = np.random.default_rng(v)
    raw, sym, opt, post = _cases(rng, 8, net.row_len)
    res = h.post_outputs(raw, sym, opt, post)
    pp = tuple(float(x) for x in net.desc.post_process_params)
    for i in range(8):
        q = post[i]
        ref = oracle.postprocess_row(raw[i], net.P, net.S, v, int(sym[i]), float(opt[i]), q["legal"],
                                     q["white_to_move"], q["board_x_size"], q["board_y_size"],
                                     q["nn_policy_temperature"], q["enable_passing_hacks"], q["no_result_allowed"], pp)
        _compare(res[i], ref, v, f"v{v} row {i}")
    h.close()


def test_post_outputs_edge_cases(kgx, synth, oracle):
    net = kgx.Net(synth.write_model(_arch(synth, 14), 3))
    h = kgx.Handle(net, 4, "f32")
    rng = np.random.default_rng(5)
    raw, sym, opt, post = _cases(rng, 4, net.row_len)
    pp = tuple(float(x) for x in net.desc.post_process_params)
    # The pass prior capped at 19 times the other moves: a dominant pass logit gets exactly 19 / 20.
    raw[0, 361] = 20.0  # dominant, yet the others' sum (times 19) stays above the 1e-20 floor
    raw[0, 362 + 361] = 20.0
    post[0]["enable_passing_hacks"] = True
    # A single legal move gets probability 1.
    post[1]["legal"] = np.zeros(362, np.uint8)
    post[1]["legal"][40] = 1
    res = h.post_outputs(raw, sym, opt, post)
    assert abs(res[0]["policy"][361] - 0.95) < 1e-6
    assert res[1]["policy"][40] == 1.0 and np.all(np.delete(res[1]["policy"], 40) == -1.0)
    for i in range(4):
        q = post[i]
        ref = oracle.postprocess_row(raw[i], net.P, net.S, 14, int(sym[i]), float(opt[i]), q["legal"],
                                     q["white_to_move"], q["board_x_size"], q["board_y_size"],
                                     q["nn_policy_temperature"], q["enable_passing_hacks"], q["no_result_allowed"], pp)
        _compare(res[i], ref, 14, f"edge row {i}")
    # The reference's two nonfinite errors, and the checks on the inputs.
    bad = raw.copy()
    bad[2, :362] = np.inf
    post2 = [dict(q) for q in post]
    post2[2]["legal"] = np.ones(362, np.uint8)
    with pytest.raises(kgx.KgError, match="Got nonfinite for policy sum"):
        h.post_outputs(bad, sym, opt, post2)
    bad = raw.copy()
    bad[3, net.P * 362] = np.inf
    with pytest.raises(kgx.KgError, match="Got nonfinite for nneval value"):
        h.post_outputs(bad, sym, opt, post)
    post3 = [dict(q) for q in post]
    post3[0]["legal"] = np.zeros(362, np.uint8)
    with pytest.raises(kgx.KgError, match="no legal move"):
        h.post_outputs(raw, sym, opt, post3)
    post3 = [dict(q) for q in post]
    post3[1]["board_x_size"] = 20
    with pytest.raises(kgx.KgError, match="board size"):
        h.post_outputs(raw, sym, opt, post3)
    post3 = [dict(q) for q in post]
    post3[2]["nn_policy_temperature"] = 0.0
    with pytest.raises(kgx.KgError, match="nnPolicyTemperature"):
        h.post_outputs(raw, sym, opt, post3)
    # The handle still works after the errors.
    res = h.post_outputs(raw, sym, opt, post)
    assert abs(res[0]["policy"][361] - 0.95) < 1e-6
    h.close()


@pytest.mark.parametrize("prec", ["f32", "f16"])
def test_get_output_eval_matches_forward_and_oracle(kgx, synth, oracle, prec):
    """get_output with the post-processing on the device against the same handle's raw forward rows (inputs through
    the row symmetry) post-processed by the oracle."""
    arch = synth.tiny_nets()["t_rmspos"]  # v17, P = 2
    net = kgx.Net(synth.write_model(arch, 4))
    h = kgx.Handle(net, 6, prec)
    sp, gl, _ = synth.make_inputs(6, 9, board_sizes=[19, 13, 9, 19, 13, 9])
    rng = np.random.default_rng(11)
    _, sym, opt, post = _cases(rng, 6, net.row_len)
    for i, bs in enumerate([19, 13, 9, 19, 13, 9]):
        post[i]["board_x_size"] = post[i]["board_y_size"] = bs
        off = np.array([(p // 19 >= bs or p % 19 >= bs) for p in range(361)] + [False])
        post[i]["legal"][off] = 0
    rows = [{"spatial": sp[i], "glob": gl[i], "symmetry": int(sym[i]), "policy_optimism": float(opt[i])}
            for i in range(6)]
    res = h.get_output_eval(rows, post)
    raw = h.forward(np.stack([oracle.copy_with_symmetry(sp[i:i + 1], int(sym[i]))[0] for i in range(6)]), gl)
    pp = tuple(float(x) for x in net.desc.post_process_params)
    for i in range(6):
        q = post[i]
        ref = oracle.postprocess_row(raw[i], net.P, net.S, arch.model_version, int(sym[i]), float(opt[i]),
                                     q["legal"], q["white_to_move"], q["board_x_size"], q["board_y_size"],
                                     q["nn_policy_temperature"], q["enable_passing_hacks"], q["no_result_allowed"], pp)
        _compare(res[i], ref, arch.model_version, f"eval {prec} row {i}")
    h.close()


def test_post_outputs_match_reference_skipnn_fixture(kgx, synth):
    """kg_post_outputs on the reference's own skip-NN evaluations (fixtures/upstream-v1.18.2/unit/oracle/
    nneval_skipnn.txt, regenerated by tests/golden/gen_nneval_skipnn.py; the oracle reproduces them bit for bit):
    every policy probability, value field and ownership value against the fixture, bit for bit."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "nneval_skipnn.npz"))
    net = kgx.Net(synth.write_model(synth.tiny_nets()["t_rmspos"], 4))  # model version 17, P = 2, S = 6
    assert (net.P, net.S, net.desc.model_version, net.row_len) == (2, 6, 17, 1094)
    assert tuple(float(x) for x in net.desc.post_process_params) == (20.0, 20.0, 20.0, 20.0, 40.0, 0.25, 30.0)
    n = len(z["line"])
    raw = np.zeros((n, net.row_len), np.float32)
    raw[:, :362] = z["raw_policy"]
    raw[:, 362:724] = z["raw_policy"]
    raw[:, 724:727] = z["raw_value"]
    raw[:, 727:733] = z["raw_score"]
    raw[:, 733:] = z["raw_owner"]
    post = [{"legal": z["legal"][i], "white_to_move": bool(z["white"][i]), "board_x_size": int(z["board"][i][0]),
             "board_y_size": int(z["board"][i][1]), "nn_policy_temperature": float(z["temperature"][i]),
             "enable_passing_hacks": bool(z["passing"][i]), "no_result_allowed": bool(z["no_result"][i])}
            for i in range(n)]
    h = kgx.Handle(net, n, "f32")
    res = h.post_outputs(raw, np.zeros(n, np.int64), z["optimism"].astype(np.float32), post)
    h.close()
    for i in range(n):
        exp_own = z["exp_owner"][i].view(np.float32) if z["owner"][i] else None
        ref = (0, z["exp_policy"][i].view(np.float32), z["exp_fields"][i].view(np.float32),
               exp_own if exp_own is not None else res[i]["ownership"])
        _compare(res[i], ref, 17, f"fixture line {int(z['line'][i])}")
