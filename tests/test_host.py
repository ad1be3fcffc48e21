"""Host-side checks of the product library that need no GPU: every declared entry point is exported, the model
parser agrees with the oracle's and rejects what the reference rejects, bucket choice matches the reference's
cases, and handle creation refuses unsupported contexts before touching a device."""

import gzip
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol(kgx):
    header = open(os.path.join(ROOT, "include", "kgx.h")).read()
    declared = sorted(set(re.findall(r"\b(kg_[a-z0-9_]+)\s*\(", header)))
    assert declared, "no declarations found"
    lib = kgx.lib()
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(kgx.EXPORTS) == declared


def test_library_defines_every_kernel_stub(kgx):
    """A kernel template whose host-side instantiation fails is dropped silently, leaving its launch stub
    undefined in the shared library (it would fail only when loaded with lazy binding resolved)."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    so = os.path.join(ROOT, "katago-rs_amd", "libkgx.so")
    out = subprocess.run([nm, "-D", "--undefined-only", so], capture_output=True, text=True, check=True).stdout
    assert "__device_stub__" not in out, [l for l in out.splitlines() if "__device_stub__" in l][:5]


def _device_kernels(obj, tmp):
    """(name, scratch bytes per lane, spilled VGPRs) of every gfx950 kernel in one object of the library build,
    from the code object's metadata notes."""
    import subprocess
    llvm = "/opt/rocm/llvm/bin"
    fat, co = os.path.join(tmp, "fatbin"), os.path.join(tmp, "gfx950.co")
    subprocess.run([f"{llvm}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj, os.path.join(tmp, "o")],
                   check=True, capture_output=True)
    subprocess.run([f"{llvm}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True, capture_output=True)
    notes = subprocess.run([f"{llvm}/llvm-readelf", "--notes", co], check=True, capture_output=True,
                           text=True).stdout
    names = re.findall(r"^\s+\.name:\s+(\S+)", notes, re.M)
    scratch = [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)]
    spills = [int(v) for v in re.findall(r"\.vgpr_spill_count:\s+(\d+)", notes)]
    assert len(names) == len(scratch) == len(spills), obj
    return list(zip(names, scratch, spills))


def test_kernels_use_no_scratch(tmp_path):
    """No kernel of the library spills registers to scratch memory (a spill in a hot loop costs more than the
    occupancy or tile choice that caused it)."""
    import glob
    objs = sorted(glob.glob(os.path.join(ROOT, "katago-rs_amd", "csrc", "build", "*.o")))
    if not objs or not os.path.exists("/opt/rocm/llvm/bin/clang-offload-bundler"):
        pytest.skip("library objects or ROCm LLVM tools not available")
    bad, n = [], 0
    for obj in objs:
        with open(obj, "rb") as f:
            data = f.read()
            # (an offload bundle, or a compressed one: kgx_kernels.o's is compressed)
            if b"__CLANG_OFFLOAD_BUNDLE__" not in data and b"CCOB" not in data:
                continue  # host-only object
        for name, scratch, spills in _device_kernels(obj, str(tmp_path)):
            n += 1
            if scratch or spills:
                bad.append((os.path.basename(obj), name, scratch, spills))
    assert n > 50, n
    assert not bad, bad[:5]


def _nets(synth):
    nets = dict(synth.tiny_nets())
    for name in ("b10c128", "b18c384nbt", "b10c384h6"):
        nets[name] = synth.CONFIGS[name][0]()
    return nets


def test_parser_agrees_with_oracle(kgx, synth, oracle):
    for name, arch in _nets(synth).items():
        mb = synth.write_model(arch, 5)
        net = kgx.Net(mb)
        om = oracle.Model(mb)
        assert (net.version, net.P, net.S, net.row_len, net.num_input_channels, net.num_global, net.num_meta) == \
               (om.version, om.P, om.S, om.row_len, om.num_input_channels, om.num_global, om.num_meta), name
        assert net.desc.trunk_num_channels == arch.trunk_c
        assert net.name == arch.name
        assert net.row_len == synth.row_len(arch)


def test_parser_reads_gzip_and_text_models(kgx, synth):
    arch = synth.tiny_nets()["t_tf"]
    mb, _ = synth.write_model_tree(arch, 2)
    txt, _ = synth.write_model_tree(arch, 2, text_floats=True)
    p = [kgx.Net(b).desc.num_parameters for b in (mb, gzip.compress(mb), txt)]
    assert p[0] == p[1] == p[2] > 0


def test_parser_rejections(kgx, synth):
    arch = synth.tiny_nets()["t_res"]
    mb = synth.write_model(arch, 1)
    with pytest.raises(kgx.KgError, match="expectedSha256 is not supported"):
        kgx.Net(mb, expected_sha256="00" * 32)
    with pytest.raises(kgx.KgError):
        kgx.Net(mb[: len(mb) // 2])
    with pytest.raises(kgx.KgError, match="unparsed trailing bytes"):
        kgx.Net(mb + b" 7")
    newer = mb.replace(b"t-res\n14\n", b"t-res\n18\n", 1)
    with pytest.raises(kgx.KgError, match="requires a newer KataGo version"):
        kgx.Net(newer)
    bad_kind = mb.replace(b"ordinary_block", b"mystery_block", 1)
    with pytest.raises(kgx.KgError, match="unknown block kind"):
        kgx.Net(bad_kind)
    with pytest.raises(kgx.KgError, match="Model name"):
        kgx.Net(mb.replace(b"t-res", b"t.res", 1))


def _fnv1a(a) -> int:
    """FNV-1a 64 over the little-endian bytes of float32 values (nninputs.cpp:43-45 of the reference's
    fixtures)."""
    h = 0xCBF29CE484222325
    for b in np.ascontiguousarray(a, "<f4").tobytes():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_symmetry_copies_match_reference_fixtures(kgx):
    """copy_inputs_with_symmetry / copy_outputs_with_symmetry against the reference's own oracle fixtures
    (fixtures/upstream-v1.18.2/unit/oracle/nninputs_expected.txt, via tests/golden/gen_nninputs_sym.py): 57
    featurized rows on square and non-square boards over all eight symmetries, bit-exact by FNV-1a."""
    g = np.load(os.path.join(ROOT, "tests", "golden", "nninputs_sym.npz"))
    syms = set()
    for ci, (pid, ei, sym, nx, ny) in enumerate(g["meta"]):
        bits = np.zeros(22 * nx * ny, np.uint32)
        sel = g["nz_case"] == ci
        bits[g["nz_index"][sel]] = g["nz_bits"][sel]
        row = bits.view(np.float32).reshape(22, ny, nx)
        fnv_nchw, fnv_in, fnv_out = (int(v) for v in g["hashes"][ci])
        assert _fnv1a(row) == fnv_nchw, (pid, ei)
        s = int(sym) if sym >= 0 else 0
        syms.add(s)
        assert _fnv1a(kgx.copy_with_symmetry(row, s)) == fnv_in, (pid, ei, s, nx, ny)
        assert _fnv1a(kgx.copy_with_symmetry(row[:1], s, reverse=True)) == fnv_out, (pid, ei, s, nx, ny)
    assert syms == set(range(8))


def test_symmetry_copy_rejects_bad_arguments(kgx):
    x = np.zeros((1, 3, 3), np.float32)
    with pytest.raises(kgx.KgError):
        kgx.copy_with_symmetry(x, 8)
    with pytest.raises(kgx.KgError):
        kgx.copy_with_symmetry(x, -1)


def test_padded_batch_size_reference_cases(kgx):
    # crates/katago-nn-burn/tests/batch_buckets.rs:27-35
    b = [1, 2, 4, 8, 16, 32]
    assert kgx.padded_batch_size(b, 1, 32) == 1
    assert kgx.padded_batch_size(b, 3, 32) == 4
    assert kgx.padded_batch_size(b, 17, 32) == 32
    assert kgx.padded_batch_size(b, 17, 24) == 17
    assert kgx.padded_batch_size([], 5, 32) == 5


def test_handle_rejects_unsupported_contexts(kgx, synth):
    # createComputeContext / createComputeHandle checks (backend.rs:300-372), made before any device call.
    net = kgx.Net(synth.write_model(synth.tiny_nets()["t_res"], 1))
    with pytest.raises(kgx.KgError, match="nnXLen and nnYLen must equal"):
        kgx.Handle(net, 4, "f32", nn_x_len=9, nn_y_len=9)
    with pytest.raises(kgx.KgError, match="inputsUseNHWC = true unsupported"):
        kgx.Handle(net, 4, "f32", inputs_use_nhwc=True)
    with pytest.raises(kgx.KgError, match="max batch size"):
        kgx.Handle(net, 0, "f32")


def test_synthetic_inputs_follow_the_benchmark_distribution(synth):
    sp, gl, me = synth.make_inputs(64, 0, board_sizes=[19, 9], meta=1)
    assert sp.shape == (64, 22, 19, 19) and gl.shape == (64, 19) and me.shape == (64, 192)
    assert set(np.unique(sp)) <= {0.0, 1.0}
    assert np.all(sp[0::2, 0] == 1) and sp[1, 0].sum() == 81
    assert np.all(sp[1, :, 9:, :] == 0) and np.all(sp[1, :, :, 9:] == 0)
    frac = sp[0::2, 1:].mean()
    assert 0.27 < frac < 0.33
    assert np.all(np.abs(gl[:, 5]) <= 1) and set(np.unique(np.delete(gl, 5, axis=1))) <= {0.0, 1.0}


def test_handle_entry_points_reject_a_null_handle(kgx):
    """Every entry point that takes a handle returns an error for a NULL one (no device work is started)."""
    L = kgx.lib()
    p = kgx.ctypes.c_void_p()
    calls = {
        "kg_sync": lambda: L.kg_sync(None),
        "kg_profile_enable": lambda: L.kg_profile_enable(None, 1),
        "kg_profile_reset": lambda: L.kg_profile_reset(None),
        "kg_run": lambda: L.kg_run(None, 1, None),
        "kg_forward": lambda: L.kg_forward(None, 1, None, None, None, None),
        "kg_handle_set_batch_buckets": lambda: L.kg_handle_set_batch_buckets(None, None, 0),
        "kg_handle_device_buffers": lambda: L.kg_handle_device_buffers(None, kgx.ctypes.byref(p), None, None, None),
        "kg_get_output": lambda: L.kg_get_output(None, 1, None, None),
        "kg_get_output_async": lambda: L.kg_get_output_async(None, 1, None, None, kgx.DONE_FN(0), None),
        "kg_wait": lambda: L.kg_wait(None),
        "kg_run_static": lambda: L.kg_run_static(None, 1),
    }
    for name, call in calls.items():
        assert call() != 0, name
        err = L.kg_last_error().decode()
        assert "null handle" in err, (name, err)
    assert L.kg_profile_read(None, None, None, None, None, None, 0) == -1
    assert L.kg_handle_stream(None) is None
    assert L.kg_handle_is_using_fp16(None) == 0


def test_copy_outputs_sentinels_follow_every_reference_branch(kgx):
    """kg_copy_outputs on rows of distinct sentinel values: every field comes from the slot copy_outputs reads
    (backend.rs:622-731), for every model-version branch and policy channel count, at optimism 0 (channel 0
    exactly), 1 (channel 1 exactly) and 0.25, with the pass logits at c * 362 + 361 and the inverse symmetry."""
    import outputs_spec as spec
    for v, P in spec.CASES:
        S = spec.score_channels(v)
        raw = spec.sentinel_row(P, S)
        for opt in spec.OPTIMISMS:
            pol, fields, own = spec.expected(raw, P, S, v, opt)
            if opt in (0.0, 1.0) and (P == 2 or (P == 4 and v >= 16)):
                c = int(opt)  # exact: the row's own channel c, pass logit included
                assert np.array_equal(pol, raw[c * 362:(c + 1) * 362]), (v, P, opt)
            for sym in (0, 3, 5):
                res = kgx.copy_outputs(raw[None], P, S, v, sym, opt)[0]
                want_pol = np.append(kgx.copy_with_symmetry(pol[:361].reshape(1, 19, 19), sym, reverse=True).ravel(),
                                     pol[361])
                assert np.array_equal(res["policy"], want_pol), (v, P, opt, sym)
                got = np.array([res[k] for k in spec.FIELDS], np.float32)
                assert np.array_equal(got, fields), (v, P, opt, sym, got, fields)
                want_own = kgx.copy_with_symmetry(own.reshape(1, 19, 19), sym, reverse=True).ravel()
                assert np.array_equal(res["ownership"], want_own), (v, P, opt, sym)
    with pytest.raises(kgx.KgError, match="score value channels"):
        kgx.copy_outputs(spec.sentinel_row(1, 4)[None], 1, 4, 9, 0, 0.0)
    with pytest.raises(kgx.KgError, match="symmetry"):
        kgx.copy_outputs(spec.sentinel_row(1, 6)[None], 1, 6, 9, 8, 0.0)


def test_model_version_table_matches_reference_fixture(kgx):
    """NNModelVersion's per-version input layout against KataGo's own outputs
    (fixtures/upstream-v1.18.2/unit/oracle/modelversion_desc.txt, extracted by tests/golden/gen_modelversion.py):
    values for versions 3..17, the reference's error text for -2..2 and 18..20, and the meta encoder channels."""
    import json
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "modelversion_desc.json")))
    idx = {"getInputsVersion": 0, "getNumSpatialFeatures": 1, "getNumGlobalFeatures": 2}
    n = 0
    for e in fx["V"]:
        fn, arg = e["fn"], e["arg"]
        call = (lambda a=arg: kgx.model_version_features(a)[idx[fn]]) if fn in idx else \
            (lambda a=arg: kgx.meta_encoder_channels(a))
        if "err" in e:
            with pytest.raises(kgx.KgError) as ei:
                call()
            assert str(ei.value) == e["err"], (fn, arg)
        else:
            assert call() == e["value"], (fn, arg)
        n += 1
    assert n == 74


def test_model_post_process_defaults_match_reference_fixture(kgx, synth):
    """A model before version 13 stores no post-process parameters: the desc carries ModelPostProcessParams'
    defaults, which the reference's fixture pins (P lines of modelversion_desc.txt)."""
    import json
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "modelversion_desc.json")))["P"]
    net = kgx.Net(synth.write_model(synth.tiny_nets()["t_v8"], 1))
    names = ["tdScoreMultiplier", "scoreMeanMultiplier", "scoreStdevMultiplier", "leadMultiplier",
             "varianceTimeMultiplier", "shorttermValueErrorMultiplier", "shorttermScoreErrorMultiplier"]
    assert list(net.desc.post_process_params) == [fx[k] for k in names]


def test_handle_rejects_input_counts_of_another_model_version(kgx, synth):
    """BurnInputBuffers::new asserts the model's input channels against its version (backend.rs:184-188); the
    handle refuses such a model before touching a device."""
    arch = synth.tiny_nets()["t_res"]
    arch.num_global_channels = 18
    net = kgx.Net(synth.write_model(arch, 1))
    with pytest.raises(kgx.KgError, match="model version 14 takes 22 spatial and 19 global input features"):
        kgx.Handle(net, 2, "f16")
