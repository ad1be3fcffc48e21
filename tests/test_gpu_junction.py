"""The nested-bottleneck junction (one block's exit 1x1 convolution, 192 -> 384 into the trunk, and the next block's
entry 1x1, 384 -> 192, in one launch: launch_junction, kgx_junction.hip), and the head junction (the last block's
exit and the heads' p1 | g1 | v1 1x1, 384 -> 96, where the trunk ends and is not written), and the stem junction
(the network's stem, a 3x3 convolution of the packed input into the trunk, and the first block's entry 1x1), through
the C ABI:
- bit for bit equal to the two separate split-operand launches it replaces (KGX_JUNCTION=0 plans those), on f16 and
  bf16 handles, at a ragged batch (tiles past the last pixel) and at batch 32, with gpool inner blocks between, for
  mish nets and (the run-time activation kernel) ReLU nets;
- the junction net against the float64 oracle and the 16-bit network (the bounds of test_gpu_parity.py);
- the planning: a net of n nested blocks over 384 / 192 channels runs a stem junction, n - 1 junctions, one head
  junction and no separate 1x1 or stem convolution."""

import numpy as np
import pytest

from test_gpu_parity import check, emulated

pytestmark = pytest.mark.gpu


def junction_arch(synth, n=3, act="ACTIVATION_MISH"):
    inner = [[("res", 192)], [("gpool", 192, 64), ("res", 192)], [("res", 192), ("res", 192)]]
    return synth.Arch("t-junction", 14, 384, [("nbt", 192, inner[k % 3]) for k in range(n)], mid_c=192, gpool_c=64,
                      act=act)


def run(kgx, mb, batch, prec, sp, gl, monkeypatch, junction):
    if junction:
        monkeypatch.delenv("KGX_JUNCTION", raising=False)
    else:
        monkeypatch.setenv("KGX_JUNCTION", "0")
    net = kgx.Net(mb)
    h = kgx.Handle(net, batch, prec)
    h.profile(True)
    h.profile_reset()
    out = h.forward(sp, gl)
    prof = h.profile_read()
    h.profile(False)
    again = h.forward(sp, gl)  # graph replay
    h.close()
    assert np.array_equal(out, again)
    return out, prof, net


@pytest.mark.parametrize("prec,batch,act", [("f16", 5, "ACTIVATION_MISH"), ("bf16", 5, "ACTIVATION_MISH"),
                                            ("f16", 32, "ACTIVATION_MISH"), ("bf16", 32, "ACTIVATION_MISH"),
                                            ("f16", 7, "ACTIVATION_RELU"), ("f16", 1, "ACTIVATION_MISH")])
def test_junction_equals_the_two_separate_launches(kgx, synth, monkeypatch, prec, batch, act):
    """(ReLU nets run the junction's kernel that takes the emission's activation at run time.)"""
    print(f"junction vs separate launches: {prec}, batch {batch}, {act}", flush=True)
    mb = synth.write_model(junction_arch(synth, 4, act), 7)
    sp, gl, _ = synth.make_inputs(batch, 11, board_sizes=[19, 19, 13, 9, 19, 7])
    fused, pf, _ = run(kgx, mb, batch, prec, sp, gl, monkeypatch, True)
    sep, ps, _ = run(kgx, mb, batch, prec, sp, gl, monkeypatch, False)
    assert pf["conv1x1_junction"]["launches"] == 3 and "conv1x1_junction" not in ps
    assert pf["head_junction"]["launches"] == 1 and "head_1x1" not in pf
    assert ps["head_1x1"]["launches"] == 1 and "head_junction" not in ps
    assert pf["stem_junction"]["launches"] == 1 and "conv3x3_n96" not in pf
    assert ps["conv3x3_n96"]["launches"] == 1 and "stem_junction" not in ps
    # the separate plan's 1x1s: four entries and four exits; the junction plan keeps none
    sep_1x1 = sum(v["launches"] for k, v in ps.items() if k.startswith("conv1x1_split"))
    fused_1x1 = sum(v["launches"] for k, v in pf.items() if k.startswith("conv1x1_split"))
    assert sep_1x1 == 8 and fused_1x1 == 0, (ps.keys(), pf.keys())
    assert np.all(np.isfinite(fused))
    assert np.array_equal(fused, sep), f"{prec} batch {batch}: max diff {np.abs(fused - sep).max():.3e}"


@pytest.mark.parametrize("prec", ["f16", "bf16"])
def test_junction_net_matches_oracle(kgx, synth, oracle, monkeypatch, prec):
    print(f"junction net vs oracle: {prec}", flush=True)
    mb = synth.write_model(junction_arch(synth, 3), 9)
    rows = [0, 1, 2, 3]
    sp, gl, _ = synth.make_inputs(6, 13, board_sizes=[19, 13, 9, 19, 19, 5])
    out, prof, net = run(kgx, mb, 6, prec, sp, gl, monkeypatch, True)
    assert prof["conv1x1_junction"]["launches"] == 2 and prof["head_junction"]["launches"] == 1
    assert prof["stem_junction"]["launches"] == 1
    ref = oracle.Model(mb).forward(sp[rows], gl[rows])
    check(out[rows], ref, net.P, net.S, prec, f"junction net", emulated(oracle, mb, prec, sp[rows], gl[rows]))


def test_head_junction_only_for_96_head_channels(kgx, synth, monkeypatch):
    """Heads of 64 + 32 + 32 channels keep their own 1x1 launch after the last exit, with the same bits as the
    separate plan."""
    print("junction net with 128 head channels", flush=True)
    arch = junction_arch(synth, 2)
    arch.p1_c = 64
    mb = synth.write_model(arch, 5)
    sp, gl, _ = synth.make_inputs(5, 3, board_sizes=[19, 13, 19, 9, 19])
    fused, pf, _ = run(kgx, mb, 5, "f16", sp, gl, monkeypatch, True)
    sep, _, _ = run(kgx, mb, 5, "f16", sp, gl, monkeypatch, False)
    assert pf["conv1x1_junction"]["launches"] == 1 and "head_junction" not in pf and pf["head_1x1"]["launches"] == 1
    assert pf["stem_junction"]["launches"] == 1
    assert sum(v["launches"] for k, v in pf.items() if k.startswith("conv1x1_split")) == 1
    assert np.array_equal(fused, sep)


def test_l2_weight_touch_changes_no_bits(kgx, synth, monkeypatch):
    """Kernels touch the next convolution's weights into L2 during their epilogue (ConvOut::pf); with the touch
    off (KGX_L2_PREFETCH=0) the outputs are the same bits."""
    print("junction net with and without the L2 weight touch", flush=True)
    mb = synth.write_model(junction_arch(synth, 3), 6)
    sp, gl, _ = synth.make_inputs(9, 4, board_sizes=[19, 13, 19, 9, 19])
    on, _, _ = run(kgx, mb, 9, "f16", sp, gl, monkeypatch, True)
    monkeypatch.setenv("KGX_L2_PREFETCH", "0")
    off, _, _ = run(kgx, mb, 9, "f16", sp, gl, monkeypatch, True)
    assert np.array_equal(on, off)
