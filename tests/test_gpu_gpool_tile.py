"""A global-pooling block's mid activation per 192-pixel tile (launch_gpool_tile, kgx_kernels.hip: the pooled
features from the gpool conv's partials, the matmul to the row bias, the emission) through the C ABI, bit for bit
equal to the per-row program it replaces (KGX_GPOOL_TILE=0 plans that one), on f16 and bf16 handles, mish and
ReLU nets, gpool blocks of 192 | 64 and 128 | 128 channels (256-output gpool convs, which pool into partials), and
a 128 | 32 block, which keeps the row program (its conv has no partials), at ragged batches (tiles that cross batch rows and tiles
past the last pixel) and at batch 32."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def gpool_arch(synth, act):
    blocks = [("gpool", 192, 64), ("res", 192), ("gpool", 128, 128), ("gpool", 128, 32), ("res", 192)]
    return synth.Arch("t-gpool-tile", 14, 192, blocks, mid_c=192, gpool_c=64, act=act)


def run(kgx, mb, batch, prec, sp, gl, monkeypatch, tile):
    if tile:
        monkeypatch.delenv("KGX_GPOOL_TILE", raising=False)
    else:
        monkeypatch.setenv("KGX_GPOOL_TILE", "0")
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
    return out, prof


@pytest.mark.parametrize("prec,batch,act", [("f16", 5, "ACTIVATION_MISH"), ("bf16", 7, "ACTIVATION_MISH"),
                                            ("f16", 32, "ACTIVATION_MISH"), ("f16", 3, "ACTIVATION_RELU"),
                                            ("f16", 1, "ACTIVATION_MISH")])
def test_gpool_tile_equals_the_row_program(kgx, synth, monkeypatch, prec, batch, act):
    print(f"gpool tile vs row program: {prec}, batch {batch}, {act}", flush=True)
    mb = synth.write_model(gpool_arch(synth, act), 12)
    sp, gl, _ = synth.make_inputs(batch, 17, board_sizes=[19, 13, 19, 9, 19, 7, 19])
    tiled, pt = run(kgx, mb, batch, prec, sp, gl, monkeypatch, True)
    rows, pr = run(kgx, mb, batch, prec, sp, gl, monkeypatch, False)
    assert pt["gpool_tile"]["launches"] == 2 and pt["row_prog_gpool"]["launches"] == 1, pt.keys()
    assert pr["row_prog_gpool"]["launches"] == 3 and "gpool_tile" not in pr, pr.keys()
    assert np.all(np.isfinite(tiled))
    assert np.array_equal(tiled, rows), f"{prec} batch {batch}: max diff {np.abs(tiled - rows).max():.3e}"
