"""Parity of the HIP forward pass (through the C ABI) with the float64 CPU oracle, on the device.

Tolerances, per output group (policy, value, score, ownership) of each row block, with no allowance:
- f32: max |gpu - oracle| <= 1e-4 * max |oracle| over the group (the f32 tier's 1e-4 relative error);
- f16: max |gpu - oracle| <= 2e-2 absolute;
- bf16: max |gpu - oracle| <= 1.6e-1 absolute: the f16 bound scaled by 8, the ratio of the two types' unit
  roundoffs (2^-8 against 2^-11; no reference tier exists for bf16).
16-bit handles round the operands of their 3x3 convolutions (stem included) and of the transformer token GEMMs
and attention; the 1x1 convolutions of the trunk run on split (high + low) 16-bit operands, float-accurate, as
the reference's f16 mode keeps them in float (crates/katago-nn-burn/src/backend.rs:399-403). They are also held
to the "16-bit network", the oracle evaluated with the same operands rounded at the same points:
max |gpu - emulation| <= 2 x the format's own error (emulation against float64) + 1e-4 * max(1, max |oracle|).
Index work (symmetry, padding rows, batch buckets, tile scatter) is checked bit-exactly where the arithmetic
is identical: a row's outputs must not depend on the batch it runs in, nor on its position in it.
"""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {"f32": ("rel", 1e-4), "f16": ("abs", 2e-2), "bf16": ("abs", 1.6e-1)}
# The layer classes whose operands 16-bit handles round (oracle.QCLASS): all but the nested-bottleneck 1x1s.
ROUNDED = ("stem", "conv3", "gconv", "token")


def groups(P, S):
    p = P * 362
    return {"policy": slice(0, p), "value": slice(p, p + 3), "score": slice(p + 3, p + 3 + S),
            "ownership": slice(p + 3 + S, p + 3 + S + 361)}


def errors(out, ref, P, S):
    res = {}
    for k, sl in groups(P, S).items():
        d = np.abs(out[:, sl].astype(np.float64) - ref[:, sl])
        res[k] = (float(d.max()), float(np.abs(ref[:, sl]).max()))
    return res


def check(out, ref, P, S, prec, what, ref_q=None):
    """ref: the float64 oracle; ref_q (16-bit handles): the oracle with the same 16-bit operand rounding."""
    assert np.all(np.isfinite(out)), f"{what}: non-finite outputs"
    kind, tol = TOL[prec]
    errs = errors(out, ref, P, S)
    print(f"{what} [{prec}] " + " ".join(f"{k}: err {e:.2e} (|ref| {s:.2e})" for k, (e, s) in errs.items()))
    fmt = {k: 0.0 for k in errs}
    if ref_q is not None:
        fmt = {k: e for k, (e, _) in errors(ref_q, ref, P, S).items()}
        eq = errors(out, ref_q, P, S)
        print(f"{what} [{prec}] vs {prec} network: " + " ".join(f"{k}: {e:.2e} (format {fmt[k]:.2e})" for k, (e, _) in eq.items()))
        for k, (e, s) in eq.items():
            bound = 2.0 * fmt[k] + 1e-4 * max(1.0, s)
            assert e <= bound, f"{what} [{prec}] {k}: max |gpu - {prec} network| {e:.3e} > {bound:.3e}"
    for k, (e, s) in errs.items():
        bound = tol * max(s, 1e-30) if kind == "rel" else tol
        assert e <= bound, f"{what} [{prec}] {k}: max err {e:.3e} > {bound:.3e} (|ref| max {s:.3e})"


def emulated(oracle, model_bytes, prec, spatial, glob, meta=None):
    """The oracle with the 16-bit handle's operand rounding (None for f32)."""
    if prec == "f32":
        return None
    return oracle.Model(model_bytes).forward(spatial, glob, meta, operands=prec, classes=ROUNDED)


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "oracle_tiny.npz")), np.load(os.path.join(GOLDEN, "m0_inputs.npz"))


@pytest.mark.parametrize("prec", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name", ["t_res", "t_nbt", "t_v8", "t_tf", "t_tf64", "t_human", "t_rms", "t_rmspos"])
def test_tiny_nets_match_oracle(kgx, synth, oracle, golden, name, prec):
    g, m0 = golden
    arch = synth.tiny_nets()[name]
    mb = synth.write_model(arch, 1)
    net = kgx.Net(mb)
    h = kgx.Handle(net, 8, prec)
    meta = g[f"{name}.meta"] if f"{name}.meta" in g else None
    out = h.forward(g[f"{name}.spatial"], g[f"{name}.glob"], meta)
    check(out, g[f"{name}.out"], net.P, net.S, prec, name,
          emulated(oracle, mb, prec, g[f"{name}.spatial"], g[f"{name}.glob"], meta))
    m0meta = m0["meta"] if arch.meta_encoder else None
    out = h.forward(m0["spatial"], m0["glob"], m0meta)
    check(out, g[f"{name}.m0_out"], net.P, net.S, prec, name + " m0",
          emulated(oracle, mb, prec, m0["spatial"], m0["glob"], m0meta))
    h.close()


@pytest.mark.parametrize("conv,prec", [("wino2", "f32"), ("wino2", "f16"), ("wino2", "bf16"), ("wino4", "f16")])
@pytest.mark.parametrize("name", ["t_res", "t_nbt", "t_v8"])
def test_winograd_variants_match_oracle(kgx, synth, oracle, golden, monkeypatch, name, conv, prec):
    """The Winograd kernels on every precision (16-bit handles default to the implicit GEMM, float ones to
    F(4x4,3x3)); the algorithm is chosen when the handle builds its network."""
    monkeypatch.setenv("KGX_CONV", conv)
    g, _ = golden
    mb = synth.write_model(synth.tiny_nets()[name], 1)
    net = kgx.Net(mb)
    h = kgx.Handle(net, 8, prec)
    out = h.forward(g[f"{name}.spatial"], g[f"{name}.glob"])
    if conv == "wino4" and prec != "f32":
        # F(4x4,3x3) transforms grow values up to 10x, so 16-bit operands lose about a digit (measured 3.5e-2 on
        # these nets): the reason 16-bit handles use F(2x2,3x3) or the implicit GEMM. Held to 6e-2 here.
        errs = errors(out, g[f"{name}.out"], net.P, net.S)
        assert np.all(np.isfinite(out)) and all(e <= 6e-2 for e, _ in errs.values()), errs
    else:
        # Winograd transforms round their transformed operands, not the activations: only the float64 bound.
        check(out, g[f"{name}.out"], net.P, net.S, prec, f"{name} {conv}")
    h.close()


def test_winograd_f2_benchmark_config(kgx, synth, oracle, monkeypatch):
    monkeypatch.setenv("KGX_CONV", "wino2")
    arch_fn, batch = synth.CONFIGS["b10c128"]
    mb = synth.write_model(arch_fn(), synth.CONFIG_SEEDS["b10c128"])
    sp, gl, _ = synth.make_inputs(batch, 17, board_sizes=[19, 19, 13, 9])
    net = kgx.Net(mb)
    h = kgx.Handle(net, batch, "f16")
    out = h.forward(sp, gl)
    check(out, oracle.Model(mb).forward(sp, gl), net.P, net.S, "f16", "b10c128 wino2")
    h.close()


# Rows compared with the oracle in every benchmark batch: boards 19, 19, 13 and 9 (make_inputs cycles the sizes),
# so masked pooling, masked attention keys and partial-board row programs are checked at the configs' shapes.
CONFIG_ROWS = [0, 1, 2, 3]
CONFIGS = ["b10c128", "b18c384nbt", "b10c384h6", "b10c512h8", "tf3-b11c768"]
# bf16 handles run the f16 kernels' bf16 instantiations; the headline net covers those of its shapes.
CONFIG_CASES = [(n, p) for n in CONFIGS for p in ("f32", "f16")] + [("b18c384nbt", "bf16")]


@pytest.mark.parametrize("name,prec", CONFIG_CASES)
def test_benchmark_configs_match_oracle(kgx, synth, oracle, name, prec):
    arch_fn, batch = synth.CONFIGS[name]
    mb = synth.write_model(arch_fn(), synth.CONFIG_SEEDS[name])
    rows = CONFIG_ROWS
    sp, gl, _ = synth.make_inputs(batch, 17, board_sizes=[19, 19, 13, 9])
    net = kgx.Net(mb)
    h = kgx.Handle(net, batch, prec)
    out = h.forward(sp, gl)
    ref = oracle.Model(mb).forward(sp[rows], gl[rows])
    check(out[rows], ref, net.P, net.S, prec, name, emulated(oracle, mb, prec, sp[rows], gl[rows]))
    assert np.all(np.isfinite(out))
    # Row independence over the whole batch (crates/katago-nn-burn/tests/batch_buckets.rs:98-120): the rows
    # [k:] run alone, at other offsets of every pixel tile, equal the full batch's rows bit for bit.
    for k in (1, 3, batch // 2 + 1, batch - 1):
        again = h.forward(sp[k:], gl[k:])
        assert np.array_equal(again, out[k:]), f"{name} [{prec}]: rows {k}: differ when run alone"
    h.close()


@pytest.mark.parametrize("name,prec", [(n, p) for n in ("b10c128", "b18c384nbt") for p in ("f32", "f16")])
def test_benchmark_nets_on_reference_positions(kgx, synth, oracle, name, prec):
    """The 26 featurized positions of the reference's raw-output fixtures (fixtures/m0/*.bin_input.f32 and
    *.global_input.f32: 20 positions on 19x19 boards, four on 9x9, two on 13x13), through the benchmark nets,
    against the oracle."""
    m0 = np.load(os.path.join(GOLDEN, "m0_all.npz"))
    arch_fn, _ = synth.CONFIGS[name]
    mb = synth.write_model(arch_fn(), synth.CONFIG_SEEDS[name])
    sp, gl = m0["spatial"], m0["glob"]
    net = kgx.Net(mb)
    h = kgx.Handle(net, len(sp), prec)
    out = h.forward(sp, gl)
    check(out, oracle.Model(mb).forward(sp, gl), net.P, net.S, prec, name + " m0",
          emulated(oracle, mb, prec, sp, gl))
    h.close()


@pytest.mark.parametrize("prec", ["f16", "bf16"])
@pytest.mark.parametrize("qk_gain", [3.0, 6.0])
def test_sharp_attention_matches_the_16bit_network(kgx, synth, oracle, prec, qk_gain):
    """Attention with large score ranges: the q and k projections scaled by qk_gain (scores by its square), so
    that a query's running maximum jumps by many binary orders between key tiles and the 16-bit attention kernel's
    lazy rescale (the reference maximum moves only when a numerator would exceed 2^8) takes both branches, on full
    and partial boards. Held to the 16-bit network (the oracle with the same operand rounding) with the emulation
    bound; the absolute f16 bound does not apply, since the rounding of such sharp scores moves the network
    itself far from float64."""
    import dataclasses
    arch = dataclasses.replace(synth.tiny_nets()["t_tf64"], qk_gain=qk_gain)
    mb = synth.write_model(arch, 7)
    sp, gl, _ = synth.make_inputs(6, 13, board_sizes=[19, 13, 9, 19, 7, 19])
    net = kgx.Net(mb)
    h = kgx.Handle(net, 6, prec)
    out = h.forward(sp, gl)
    h.close()
    ref = oracle.Model(mb).forward(sp, gl)
    ref_q = emulated(oracle, mb, prec, sp, gl)
    assert np.all(np.isfinite(out))
    fmt = errors(ref_q, ref, net.P, net.S)
    for k, (e, s) in errors(out, ref_q, net.P, net.S).items():
        bound = 2.0 * fmt[k][0] + 1e-4 * max(1.0, s)
        print(f"qk_gain {qk_gain} [{prec}] {k}: |gpu - {prec} network| {e:.2e}, format {fmt[k][0]:.2e}")
        assert e <= bound, f"qk_gain {qk_gain} [{prec}] {k}: {e:.3e} > {bound:.3e}"


@pytest.mark.parametrize("prec", ["f32", "f16"])
@pytest.mark.parametrize("p1,v1", [(48, 64), (96, 80)])
def test_head_widths_match_oracle(kgx, synth, oracle, p1, v1, prec):
    """Policy and value heads wider than the configs' 32 channels: the spatial heads' lanes then hold 4 and 8
    channels each (head_spatial_kernel's HK), and the row programs pool 48 to 96 channels in one or two chunks;
    against the oracle."""
    import dataclasses
    print(f"heads p1 {p1} v1 {v1} [{prec}]", flush=True)
    arch = dataclasses.replace(synth.tiny_nets()["t_res"], p1_c=p1, v1_c=v1)
    mb = synth.write_model(arch, 4)
    sp, gl, _ = synth.make_inputs(6, 8, board_sizes=[19, 13, 9, 19, 7, 19])
    net = kgx.Net(mb)
    h = kgx.Handle(net, 6, prec)
    h.profile(True)
    h.profile_reset()
    out = h.forward(sp, gl)
    prof = h.profile_read()
    h.profile(False)
    h.close()
    assert prof["row_prog_heads"]["launches"] == 1 and prof["head"]["launches"] == 1, prof.keys()
    check(out, oracle.Model(mb).forward(sp, gl), net.P, net.S, prec, f"heads {p1}/{v1}",
          emulated(oracle, mb, prec, sp, gl))


@pytest.mark.parametrize("prec", ["f16", "bf16"])
def test_mish_at_extreme_inputs_matches_the_16bit_network(kgx, synth, oracle, prec):
    """16-bit emissions compute mish as b - 2 b q with b = a * mask, q = 1 / (e (e + 2) + 2), e = exp(a), with no
    clamp or select: for a above 88.7, e overflows to infinity and q to 0, leaving b; for large negative a the two
    terms cancel. The residual blocks' mid batch norm scaled 50x drives the second convolution's input activation
    to |a| of about a hundred, so both regions occur on every board. Held to the 16-bit network (the oracle with
    the same operand rounding) with the emulation bound, outputs finite; the absolute f16 bound does not apply to a
    network this far from unit scale."""
    import dataclasses
    arch = dataclasses.replace(synth.tiny_nets()["t_res"], mid_bn_gain=50.0)
    mb = synth.write_model(arch, 9)
    sp, gl, _ = synth.make_inputs(5, 21, board_sizes=[19, 13, 9, 19, 7])
    net = kgx.Net(mb)
    h = kgx.Handle(net, 5, prec)
    out = h.forward(sp, gl)
    h.close()
    ref = oracle.Model(mb).forward(sp, gl)
    ref_q = emulated(oracle, mb, prec, sp, gl)
    assert np.all(np.isfinite(out))
    fmt = errors(ref_q, ref, net.P, net.S)
    for k, (e, s) in errors(out, ref_q, net.P, net.S).items():
        bound = 2.0 * fmt[k][0] + 1e-4 * max(1.0, s)
        print(f"mid bn x50 [{prec}] {k}: |gpu - {prec} network| {e:.2e}, format {fmt[k][0]:.2e}, |ref| {s:.2e}")
        assert e <= bound, f"mid bn x50 [{prec}] {k}: {e:.3e} > {bound:.3e}"


@pytest.mark.parametrize("prec", ["f16", "bf16"])
def test_gpool_widths_the_row_emission_does_not_fit(kgx, synth, oracle, prec):
    """A global-pooling block whose regular width has no share of a multiple of 8 channels (20): 16-bit handles
    then emit the biased mid activation with a separate bias_act launch instead of in the row program."""
    arch = synth.Arch("t-gp20", 14, 32, [("res", 32), ("gpool", 20, 16), ("res", 32)], gpool_c=16,
                      p1_c=16, g1_c=16, v1_c=16, v2_c=24)
    mb = synth.write_model(arch, 3)
    sp, gl, _ = synth.make_inputs(4, 11, board_sizes=[19, 13, 9, 19])
    net = kgx.Net(mb)
    h = kgx.Handle(net, 4, prec)
    out = h.forward(sp, gl)
    check(out, oracle.Model(mb).forward(sp, gl), net.P, net.S, prec, "t-gp20", emulated(oracle, mb, prec, sp, gl))
    h.close()


@pytest.mark.parametrize("prec", ["f16", "bf16"])
@pytest.mark.parametrize("cr,cg", [(224, 32), (128, 128), (160, 64)])
def test_gpool_conv_pooling_partials(kgx, synth, oracle, prec, cr, cg):
    """A global-pooling block whose joint 3x3 (cr + cg outputs) runs on 64-column tiles: with 256 outputs its
    pooled branch is reduced to per-tile partials in the convolution's epilogue (the filters interleaved per tile:
    56 regular + 8 pooled, or 32 + 32 columns each), with 224 the row program pools the stored branch. Oracle
    parity on ragged boards, and rows that equal the full batch's bit for bit at other offsets of the 192-pixel
    tiles."""
    arch = synth.Arch(f"t-gp{cr}-{cg}", 14, 64, [("res", 64), ("gpool", cr, cg), ("res", 64)], gpool_c=cg,
                      p1_c=16, g1_c=16, v1_c=16, v2_c=24)
    mb = synth.write_model(arch, 5)
    sp, gl, _ = synth.make_inputs(7, 12, board_sizes=[19, 13, 9, 19, 7, 19, 11])
    net = kgx.Net(mb)
    h = kgx.Handle(net, 7, prec)
    out = h.forward(sp, gl)
    check(out, oracle.Model(mb).forward(sp, gl), net.P, net.S, prec, arch.name, emulated(oracle, mb, prec, sp, gl))
    for k in (1, 2, 4):
        assert np.array_equal(h.forward(sp[k:], gl[k:]), out[k:]), f"{arch.name} [{prec}]: rows {k}:"
    h.close()


def test_rows_do_not_depend_on_batch_or_bucket(kgx, synth):
    arch = synth.tiny_nets()["t_nbt"]
    net = kgx.Net(synth.write_model(arch, 3))
    h = kgx.Handle(net, 16, "f16")
    sp, gl, _ = synth.make_inputs(16, 4, board_sizes=[19, 13, 9, 5])
    full = h.forward(sp, gl)
    for n in (1, 3, 7, 16):
        assert np.array_equal(h.forward(sp[:n], gl[:n]), full[:n]), n
    # Buckets pad with stale rows (backend.rs:549-556); the real rows are unchanged.
    h.set_batch_buckets([4, 8, 16])
    for n in (1, 3, 5):
        assert np.array_equal(h.forward(sp[:n], gl[:n]), full[:n]), n
    h.close()


def test_graph_replays_are_deterministic(kgx, synth):
    arch = synth.tiny_nets()["t_tf"]
    net = kgx.Net(synth.write_model(arch, 3))
    h = kgx.Handle(net, 8, "f16")
    sp, gl, _ = synth.make_inputs(8, 6)
    first = h.forward(sp, gl)
    for n in (8, 2, 8, 5, 8):
        out = h.forward(sp[:n], gl[:n])
        assert np.array_equal(out, first[:n])
    h.close()


def test_handles_in_flight_match_sequential(kgx, synth, oracle):
    """Several handles of one net, each driven by its own thread (the reference's serve tasks in flight,
    backend.rs:598-605): every handle's outputs equal the same handle's outputs run alone."""
    import threading
    arch = synth.tiny_nets()["t_nbt"]
    net = kgx.Net(synth.write_model(arch, 4))
    hs = [kgx.Handle(net, 8, "f16") for _ in range(3)]
    inputs = [synth.make_inputs(8, 20 + i) for i in range(3)]
    alone = [h.forward(sp, gl) for h, (sp, gl, _) in zip(hs, inputs)]
    got = [[] for _ in hs]

    def drive(i):
        sp, gl, _ = inputs[i]
        for _ in range(20):
            got[i].append(hs[i].forward(sp, gl))

    ths = [threading.Thread(target=drive, args=(i,)) for i in range(3)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    for i in range(3):
        assert len(got[i]) == 20
        for out in got[i]:
            assert np.array_equal(out, alone[i]), i
    # and what each handle returns is the network's output (the oracle, at the f16 tier).
    mb = synth.write_model(arch, 4)
    for i, (sp, gl, _) in enumerate(inputs):
        check(alone[i], oracle.Model(mb).forward(sp, gl), net.P, net.S, "f16", f"in flight {i}",
              emulated(oracle, mb, "f16", sp, gl))
    for h in hs:
        h.close()


def test_get_output_async_reads_back_on_a_helper_thread(kgx, synth, oracle):
    """kg_get_output_async (read_on_helper_thread, backend.rs:743-753): the call returns with the batch enqueued,
    a helper thread runs copy_outputs and calls back; the result equals kg_get_output's and the oracle's
    copy_outputs of the raw rows; a second call on the handle waits for the first."""
    import threading
    arch = synth.tiny_nets()["t_rms"]  # P = 4, model version 17
    net = kgx.Net(synth.write_model(arch, 8))
    h = kgx.Handle(net, 8, "f32")
    sp, gl, _ = synth.make_inputs(8, 5, board_sizes=[19, 13, 9])
    rows = [{"spatial": sp[i], "glob": gl[i], "symmetry": (3 * i) % 8, "policy_optimism": 0.5 * (i % 3)}
            for i in range(8)]
    calls = []
    p1 = h.get_output_async(rows, done=lambda st: calls.append((st, threading.get_ident())))
    p2 = h.get_output_async(rows[:3])  # joins the first call's helper before reusing the buffers
    res2 = p2.wait()
    res1 = p1.wait()
    assert len(calls) == 1 and calls[0][0] == 0 and calls[0][1] != threading.get_ident()
    sync = h.get_output(rows)
    raw = h.forward(np.stack([oracle.copy_with_symmetry(sp[i:i + 1], rows[i]["symmetry"])[0] for i in range(8)]), gl)
    for i in range(8):
        pol, fields, own = oracle.copy_outputs_row(raw[i], net.P, net.S, net.version, rows[i]["symmetry"],
                                                   rows[i]["policy_optimism"])
        for res in (res1, sync) + ((res2,) if i < 3 else ()):
            assert np.array_equal(res[i]["policy"], pol), i
            assert np.array_equal(res[i]["ownership"], own), i
            got = np.array([res[i][k] for k in ("white_win_prob", "white_loss_prob", "white_no_result_prob",
                                                "white_score_mean", "white_score_mean_sq", "white_lead",
                                                "var_time_left", "shortterm_winloss_error",
                                                "shortterm_score_error")], np.float32)
            assert np.array_equal(got, fields), i
    with pytest.raises(kgx.KgError, match="symmetry"):
        h.get_output_async([dict(rows[0], symmetry=9)])
    h.close()


def test_get_output_applies_symmetry_and_optimism(kgx, synth, oracle):
    arch = synth.tiny_nets()["t_rms"]  # P = 4 at model version 17: the optimism mix uses channels 0 and 1
    mb = synth.write_model(arch, 8)
    net = kgx.Net(mb)
    h = kgx.Handle(net, 8, "f32")
    sp, gl, _ = synth.make_inputs(8, 2, board_sizes=[19, 13])
    rows = [{"spatial": sp[i], "glob": gl[i], "symmetry": i, "policy_optimism": 0.25 * (i % 3)} for i in range(8)]
    res = h.get_output(rows)
    # Expected: the raw forward on the symmetrized inputs, then the oracle's copy_outputs.
    sym_in = np.stack([oracle.copy_with_symmetry(sp[i:i + 1], i)[0] for i in range(8)])
    raw = h.forward(sym_in, gl)
    for i in range(8):
        pol, fields, own = oracle.copy_outputs_row(raw[i], net.P, net.S, net.version, i, 0.25 * (i % 3))
        assert np.array_equal(res[i]["policy"], pol), i
        assert np.array_equal(res[i]["ownership"], own), i
        got = [res[i][k] for k in ("white_win_prob", "white_loss_prob", "white_no_result_prob", "white_score_mean",
                                   "white_score_mean_sq", "white_lead", "var_time_left", "shortterm_winloss_error",
                                   "shortterm_score_error")]
        assert np.array_equal(np.array(got, np.float32), fields), i
    h.close()


def test_old_model_version_output_unpacking(kgx, synth, oracle):
    arch = synth.tiny_nets()["t_v8"]  # P = 1, S = 4
    net = kgx.Net(synth.write_model(arch, 8))
    h = kgx.Handle(net, 2, "f32")
    sp, gl, _ = synth.make_inputs(2, 2)
    res = h.get_output([{"spatial": sp[i], "glob": gl[i], "symmetry": 5 + i, "policy_optimism": 1.0}
                        for i in range(2)])
    raw = h.forward(np.stack([oracle.copy_with_symmetry(sp[i:i + 1], 5 + i)[0] for i in range(2)]), gl)
    for i in range(2):
        pol, fields, own = oracle.copy_outputs_row(raw[i], 1, 4, 8, 5 + i, 1.0)
        assert np.array_equal(res[i]["policy"], pol)
        assert res[i]["shortterm_score_error"] == 0.0 and res[i]["var_time_left"] == fields[6]
    h.close()


def test_entry_points_reject_bad_calls(kgx, synth):
    arch = synth.tiny_nets()["t_human"]
    net = kgx.Net(synth.write_model(arch, 1))
    h = kgx.Handle(net, 4, "f16")
    sp, gl, me = synth.make_inputs(5, 1, meta=1)
    with pytest.raises(kgx.KgError, match="batch size out of range"):
        h.forward(sp, gl, me)
    with pytest.raises(kgx.KgError, match="needs a meta_input"):
        h.forward(sp[:2], gl[:2], None)
    out = h.forward(sp[:4], gl[:4], me[:4])
    assert out.shape == (4, net.row_len) and np.all(np.isfinite(out))
    h.close()


def test_device_resident_run_matches_forward(kgx, synth):
    import ctypes
    arch = synth.tiny_nets()["t_res"]
    net = kgx.Net(synth.write_model(arch, 2))
    h = kgx.Handle(net, 4, "f16")
    sp, gl, _ = synth.make_inputs(4, 3)
    ref = h.forward(sp, gl)
    h2 = kgx.Handle(net, 4, "f16")
    d_bin, d_glob, _, _ = h2.device_buffers()
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(d_bin, sp.ctypes.data, sp.nbytes, 1) == 0
    assert hip.hipMemcpy(d_glob, gl.ctypes.data, gl.nbytes, 1) == 0
    out = np.empty_like(ref)
    h2.run(4, out)
    assert np.array_equal(out, ref)
    h.close()
    h2.close()
