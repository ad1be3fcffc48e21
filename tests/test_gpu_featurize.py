"""The device featurizer (kg_featurize, kg_featurize_rows; fill_row_v7, crates/katago-core/src/neuralnet/
nninputs.rs:1336-1800, with copy_inputs' symmetry) through the C ABI, bit for bit:
- on the reference's own fixture rows (fixtures/upstream-v1.18.2/unit/oracle/nninputs_*.txt via
  tests/golden/gen_featurize.py): the FNV-1a hashes of every row in NCHW and NHWC, before and after the eval's
  symmetry, on the fixture's layouts (square and not, boards smaller than the layout), and the 19 globals;
- against the oracle (kgo_featurize, pinned by those fixtures in tests/test_featurize.py) on seeded random
  positions of every board size, all eight symmetries, both layouts, including one chain snaking over the whole
  board (the longest label propagation);
- through a handle: kg_featurize into the device input buffers, then kg_run, equals kg_forward on the oracle's rows,
  and the device buffers hold exactly the oracle's rows; kg_evaluate_positions (featurizer, forward, post-processing
  on the device) equals kg_get_output_eval on the oracle's rows, field for field."""

import ctypes

import numpy as np
import pytest

import featurize_cases as fc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def oracle():
    import oracle as o
    return o


def _oracle_row(oracle, p, nx, ny, nhwc, sym):
    row, glob = oracle.featurize(**p, nn_x=nx, nn_y=ny, nhwc=nhwc)
    shape = (1, ny, nx, 22) if nhwc else (1, 22, ny, nx)
    return oracle.copy_with_symmetry(row.reshape(shape), sym, nhwc=nhwc).reshape(-1), glob


def test_device_featurizer_matches_reference_fixture(kgx, oracle):
    cases = fc.fixture_positions()
    groups = {}
    for c in cases:
        groups.setdefault((c[1][3], c[1][4]), []).append(c)
    checked = 0
    for (nx, ny), cs in sorted(groups.items()):
        pos = kgx.make_positions([c[0] for c in cs])
        syms = [max(c[1][2], 0) for c in cs]
        for nhwc in (False, True):
            plain, glob = kgx.featurize_rows(pos, nx, ny, nhwc)
            symd, glob_s = kgx.featurize_rows(pos, nx, ny, nhwc, syms)
            assert np.array_equal(glob, glob_s)
            for i, (p, (pid, ei, sym, _, _), gbits, hashes) in enumerate(cs):
                assert fc.fnv1a(plain[i]) == hashes[1 if nhwc else 0], (pid, ei, nx, ny, nhwc)
                assert fc.fnv1a(symd[i]) == hashes[3 if nhwc else 2], (pid, ei, nx, ny, nhwc, syms[i])
                assert np.array_equal(glob[i].view(np.uint32), gbits), (pid, ei)
                want, _ = _oracle_row(oracle, p, nx, ny, nhwc, syms[i])
                assert np.array_equal(symd[i], want)
                checked += 1
    assert checked == 2 * 57


def _snake(xs, ys, pla):
    """One chain winding over the board: every other row full, joined at alternating ends."""
    color = np.zeros(361, np.uint8)
    for y in range(0, ys, 2):
        color[y * xs:(y + 1) * xs] = 1
        if y + 1 < ys:
            color[(y + 1) * xs + (xs - 1 if (y // 2) % 2 == 0 else 0)] = 1
    meta = np.array([xs, ys, pla, -1, 0, 1, 0, 0, 0, 0, 0, 0, 0], np.int32)
    z = np.zeros(361, np.uint8)
    moves = np.full(10, -2, np.int32)
    return dict(meta=meta, color=color, marks=z, area=z, enc=z, moves=moves, self_komi=7.5, pda=0.0)


def test_device_featurizer_matches_oracle_on_random_positions(kgx, oracle):
    rng = np.random.default_rng(2024)
    positions = [fc.random_position(rng, xs, ys) for xs, ys in
                 [(1, 1), (1, 19), (19, 1), (2, 2), (19, 19), (19, 19), (9, 9), (13, 13), (7, 12), (19, 18)]]
    positions += [fc.random_position(rng) for _ in range(86)]
    positions += [_snake(19, 19, 1), _snake(19, 19, 2), _snake(18, 19, 1), _snake(5, 19, 2)]
    n = len(positions)
    pos = kgx.make_positions(positions)
    for nhwc in (False, True):
        for rot in range(8):
            syms = [(i + rot) % 8 for i in range(n)]
            rows, glob = kgx.featurize_rows(pos, 19, 19, nhwc, syms)
            for i, p in enumerate(positions):
                want, wglob = _oracle_row(oracle, p, 19, 19, nhwc, syms[i])
                assert np.array_equal(rows[i], want), (i, nhwc, syms[i], p["meta"].tolist())
                assert np.array_equal(glob[i].view(np.uint32), wglob.view(np.uint32)), (i, p["meta"].tolist())
    # the snake is one chain: its liberty planes hold exactly the flood fill's count
    libs = fc.liberties_bruteforce(positions[-4]["color"], 19, 19)
    assert len(set(libs[positions[-4]["color"][:361] > 0])) == 1


def test_featurize_into_handle_then_run(kgx, synth, oracle):
    arch = synth.tiny_nets()["t_res"]  # model version 14: the version-7 inputs
    net = kgx.Net(synth.write_model(arch, 3))
    n = 6
    h = kgx.Handle(net, n, "f32")
    rng = np.random.default_rng(77)
    for call in range(2):  # two calls in a row: the second reuses the staging after the first upload
        positions = [fc.random_position(rng, 19, 19) for _ in range(n - 2)] + [fc.random_position(rng)
                                                                              for _ in range(2)]
        syms = rng.integers(0, 8, n)
        h.featurize(kgx.make_positions(positions), syms)
        out = np.empty((n, net.row_len), np.float32)
        h.run(n, out)
        rows = np.stack([_oracle_row(oracle, p, 19, 19, False, int(s))[0] for p, s in zip(positions, syms)])
        globs = np.stack([oracle.featurize(**p)[1] for p in positions])
        # the device buffers hold exactly the oracle's rows
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        d_bin, d_glob, _, _ = h.device_buffers()
        got = np.empty_like(rows)
        gotg = np.empty_like(globs)
        assert hip.hipMemcpy(got.ctypes.data, d_bin, got.nbytes, 2) == 0
        assert hip.hipMemcpy(gotg.ctypes.data, d_glob, gotg.nbytes, 2) == 0
        assert np.array_equal(got, rows) and np.array_equal(gotg, globs), call
        ref = h.forward(rows.reshape(n, 22, 19, 19), globs)
        assert np.array_equal(out, ref), call
    h.close()


def test_handle_featurize_rejects_bad_positions(kgx, synth):
    net = kgx.Net(synth.write_model(synth.tiny_nets()["t_v8"], 3))
    h = kgx.Handle(net, 2, "f32")
    p = fc.random_position(np.random.default_rng(1))
    bad = dict(p, meta=p["meta"].copy())
    bad["meta"][0] = 20
    with pytest.raises(kgx.KgError, match="board size"):
        h.featurize(kgx.make_positions([bad]))
    with pytest.raises(kgx.KgError, match="symmetry"):
        h.featurize(kgx.make_positions([p]), [9])
    with pytest.raises(kgx.KgError, match="batch size"):
        h.featurize(kgx.make_positions([p] * 3))
    h.close()


def test_all_symmetries_of_the_fixture_layouts(kgx, oracle):
    """Every symmetry on the fixture's non-square layouts (a transpose is skipped there, as in the reference)."""
    cases = fc.fixture_positions()
    for p, (pid, ei, sym, nx, ny), _, _ in cases[::7]:
        pos = kgx.make_positions([p] * 8)
        for nhwc in (False, True):
            rows, _ = kgx.featurize_rows(pos, nx, ny, nhwc, list(range(8)))
            for s, row in zip(range(8), rows):
                want, _ = _oracle_row(oracle, p, nx, ny, nhwc, s)
                assert np.array_equal(row, want), (pid, ei, nx, ny, nhwc, s)


@pytest.mark.parametrize("prec", ["f32", "f16"])
def test_evaluate_positions_equals_get_output_eval_on_oracle_rows(kgx, synth, oracle, prec):
    """Positions in, NNEvaluator's fields out, everything between on the device: the same bits as get_output_eval
    on the oracle's featurized rows (get_output applies the row symmetry to them), through a bucket larger than n."""
    arch = synth.tiny_nets()["t_rmspos"]  # model version 17: the version-7 inputs, P = 2
    net = kgx.Net(synth.write_model(arch, 4))
    h = kgx.Handle(net, 8, prec)
    h.set_batch_buckets([8])
    rng = np.random.default_rng(31)
    n = 5
    positions = [fc.random_position(rng, s, s) for s in (19, 13, 9, 19, 7)]
    sym = rng.integers(0, 8, n)
    opt = rng.uniform(0, 1, n).astype(np.float32)
    post = []
    for p in positions:
        xs, ys = int(p["meta"][0]), int(p["meta"][1])
        legal = np.zeros(362, np.uint8)
        for y in range(ys):
            for x in range(xs):
                legal[y * 19 + x] = p["color"][x + y * xs] == 0
        legal[361] = 1
        post.append({"legal": legal, "white_to_move": int(p["meta"][2]) == 2, "board_x_size": xs,
                     "board_y_size": ys, "nn_policy_temperature": 1.0, "enable_passing_hacks": False,
                     "no_result_allowed": True})
    got = h.evaluate_positions(kgx.make_positions(positions), sym, opt, post)
    rows = []
    for p, s_, o in zip(positions, sym, opt):
        row, glob = oracle.featurize(**p)
        rows.append({"spatial": row.reshape(22, 19, 19), "glob": glob, "symmetry": int(s_), "policy_optimism": float(o)})
    want = h.get_output_eval(rows, post)
    for i in range(n):
        for k in want[i]:
            a, b = np.atleast_1d(np.asarray(got[i][k])), np.atleast_1d(np.asarray(want[i][k]))
            assert a.dtype == b.dtype and a.shape == b.shape and a.tobytes() == b.tobytes(), (prec, i, k)
    h.close()
