"""The allocation-free forward pass (kg_run_static, workspace in the library's static device array) against the
ordinary one (kg_run), through the C ABI: bit-identical rows on two calls in a row, the second with fewer rows, on
nets covering the implicit-GEMM and split-operand convolutions, the Winograd path (float) and transformer blocks;
and the rejection of a batch beyond the static scratch's capacity."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    hip.hipDeviceSynchronize.argtypes = []
    return hip


def _static_vs_run(h, net, sp, gl):
    """(kg_run rows, kg_run_static rows) for the inputs sp, gl placed in the handle's device buffers."""
    hip = _hip()
    n = sp.shape[0]
    d_bin, d_glob, _, d_out = h.device_buffers()
    assert hip.hipMemcpy(d_bin, sp.ctypes.data, sp.nbytes, 1) == 0
    assert hip.hipMemcpy(d_glob, gl.ctypes.data, gl.nbytes, 1) == 0
    ref = np.empty((n, net.row_len), np.float32)
    h.run(n, ref)
    # Poison the output rows (0xff bytes are NaNs) so that the static run must write every value it returns.
    assert hip.hipMemset(d_out, 0xFF, ref.nbytes) == 0
    assert hip.hipDeviceSynchronize() == 0
    h.run_static(n)
    h.sync()
    got = np.empty_like(ref)
    assert hip.hipMemcpy(got.ctypes.data, d_out, got.nbytes, 2) == 0
    return ref, got


CASES = [("t_nbt", "f16", (8, 3)), ("t_tf", "f16", (8, 3)), ("t_res", "f32", (8, 3)), ("t_v8", "bf16", (6, 2)),
         ("b18c384nbt", "f16", (4, 2))]


@pytest.mark.parametrize("name,prec,rows", CASES)
def test_run_static_matches_run(kgx, synth, name, prec, rows):
    if name.startswith("t_"):
        arch, seed = synth.tiny_nets()[name], 5
    else:
        arch, seed = synth.CONFIGS[name][0](), synth.CONFIG_SEEDS[name]
    net = kgx.Net(synth.write_model(arch, seed))
    h = kgx.Handle(net, rows[0], prec)
    for k, n in enumerate(rows):  # two calls in a row, the second with fewer rows and other inputs
        sp, gl, _ = synth.make_inputs(n, 40 + k, board_sizes=[19, 13, 9, 19])
        ref, got = _static_vs_run(h, net, sp, gl)
        assert np.all(np.isfinite(ref))
        assert np.array_equal(got, ref), f"{name} [{prec}] {n} rows: static forward differs"
    h.close()


def test_run_static_rejects_batches_beyond_the_scratch(kgx, synth):
    """b18c384nbt's workspace for 32 rows is larger than the static scratch: the call fails before any launch."""
    arch = synth.CONFIGS["b18c384nbt"][0]()
    net = kgx.Net(synth.write_model(arch, synth.CONFIG_SEEDS["b18c384nbt"]))
    h = kgx.Handle(net, 32, "f16")
    with pytest.raises(kgx.KgError, match="out of range for the static scratch"):
        h.run_static(32)
    with pytest.raises(kgx.KgError, match="out of range"):
        h.run_static(0)
    h.close()
