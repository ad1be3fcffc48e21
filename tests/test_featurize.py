"""The featurizer's oracle (kgo_featurize, a restatement of fill_row_v7, crates/katago-core/src/neuralnet/
nninputs.rs:1336-1800) pinned by the reference's own fixtures (fixtures/upstream-v1.18.2/unit/oracle/nninputs_*.txt,
via tests/golden/gen_featurize.py):
- the 57 dumped rows: every spatial feature bit for bit, including the ones computed here from the stones (on-board,
  liberties 1/2/3); the reference's FNV-1a hashes of the whole row in NCHW and NHWC, before and after the eval's
  symmetry (square and non-square layouts, boards smaller than the layout); all 19 global features;
- all 4035 fixture evaluations: the komi clip and scaling (g5) and the komi parity wave (g18);
- liberties against an independent flood fill on seeded random boards of every size from 1x1 to 19x19."""

import numpy as np
import pytest

import featurize_cases as fc


@pytest.fixture(scope="module")
def oracle():
    import oracle as o
    return o


def test_oracle_rows_match_reference_hashes_and_globals(oracle):
    cases = fc.fixture_positions()
    assert len(cases) == 57
    for p, (pid, ei, sym, nx, ny), gbits, hashes in cases:
        row, glob = oracle.featurize(**p, nn_x=nx, nn_y=ny)
        row_h, glob_h = oracle.featurize(**p, nn_x=nx, nn_y=ny, nhwc=True)
        assert np.array_equal(glob, glob_h)
        assert np.array_equal(glob.view(np.uint32), gbits), (pid, ei, glob.view(np.uint32), gbits)
        assert fc.fnv1a(row) == hashes[0], (pid, ei, "NCHW row")
        assert fc.fnv1a(row_h) == hashes[1], (pid, ei, "NHWC row")
        s = sym if sym >= 0 else 0
        sym_n = oracle.copy_with_symmetry(row.reshape(1, 22, ny, nx), s)
        sym_h = oracle.copy_with_symmetry(row_h.reshape(1, ny, nx, 22), s, nhwc=True)
        assert fc.fnv1a(sym_n) == hashes[2], (pid, ei, s, "NCHW after symmetry")
        assert fc.fnv1a(sym_h) == hashes[3], (pid, ei, s, "NHWC after symmetry")


def test_oracle_liberty_planes_match_the_dumps(oracle):
    """Features 0 and 3-5 are computed from the stones alone: they match the fixture's dumped planes (which the
    hashes above cover too) and the liberty counts of an independent flood fill."""
    g = fc.fixture()
    for p, (pid, ei, sym, nx, ny), _, _ in fc.fixture_positions():
        xs, ys = int(p["meta"][0]), int(p["meta"][1])
        row, _ = oracle.featurize(**p, nn_x=nx, nn_y=ny)
        planes = row.reshape(22, ny, nx)
        libs = fc.liberties_bruteforce(p["color"], xs, ys).reshape(ys, xs)
        on = np.zeros((ny, nx), np.float32)
        on[:ys, :xs] = 1
        assert np.array_equal(planes[0], on)
        for k, lib in ((3, 1), (4, 2), (5, 3)):
            want = np.zeros((ny, nx), np.float32)
            want[:ys, :xs] = (libs == lib)
            assert np.array_equal(planes[k], want), (pid, ei, lib)
    assert len(g["meta"]) == 57


def test_oracle_komi_features_over_every_fixture_eval(oracle):
    """g5 (self komi clipped to +-(area + 20), over 20) and g18 (the parity wave) for all 4035 evaluations."""
    g = fc.fixture()["all_glob"]
    assert len(g) == 4035
    empty = np.zeros(361, np.uint8)
    moves = np.full(10, -2, np.int32)
    waves = set()
    for xs, ys, scoring, encore, g5, g18 in g:
        meta = [xs, ys, 1, -1, encore, 0, scoring, 0, 0, 0, 0, 0, 0]
        got = []
        for s in fc.self_komi_candidates(int(g5), int(xs * ys)):
            _, glob = oracle.featurize(meta, empty, empty, empty, empty, moves, s, 0.0, nn_x=19, nn_y=19)
            bits = glob.view(np.uint32)
            got.append((int(bits[5]), int(bits[18])))
        assert (int(g5), int(g18)) in got, (xs, ys, scoring, encore, hex(g5), hex(g18), got)
        waves.add(int(g18))
    assert len(waves) > 20  # the fixture exercises the wave well beyond its corners


def test_oracle_liberties_on_random_boards(oracle):
    rng = np.random.default_rng(11)
    sizes = [(1, 1), (1, 19), (19, 1), (2, 3), (19, 19), (9, 9), (13, 7)] + [(None, None)] * 40
    for xs, ys in sizes:
        p = fc.random_position(rng, xs, ys)
        xs, ys = int(p["meta"][0]), int(p["meta"][1])
        row, _ = oracle.featurize(**p)
        planes = row.reshape(22, 19, 19)[:, :ys, :xs]
        libs = fc.liberties_bruteforce(p["color"], xs, ys).reshape(ys, xs)
        for k, lib in ((3, 1), (4, 2), (5, 3)):
            assert np.array_equal(planes[k], (libs == lib).astype(np.float32)), (xs, ys, lib)
        stones = p["color"][:xs * ys].reshape(ys, xs)
        pla = int(p["meta"][2])
        assert np.array_equal(planes[1], (stones == pla).astype(np.float32))
        assert np.array_equal(planes[2], (stones == 3 - pla).astype(np.float32))


def test_featurize_rows_rejects_bad_positions_before_any_device_call(kgx):
    """kg_featurize_rows checks every position (the reference's asserts) before it touches a device."""
    p = fc.random_position(np.random.default_rng(3), 9, 9)
    cases = [(0, 0, "board size"), (0, 10, "outside the 9x9 layout"), (2, 3, "next_player"), (3, 81, "ko_loc"),
             (4, 3, "encore_phase"), (5, 4, "unknown rules"), (12, 6, "move history")]
    for field, value, msg in cases:
        bad = dict(p, meta=p["meta"].copy())
        bad["meta"][field] = value
        with pytest.raises(kgx.KgError, match=msg):
            kgx.featurize_rows(kgx.make_positions([bad]), 9, 9)
    bad = dict(p, color=p["color"].copy())
    bad["color"][4] = 3
    with pytest.raises(kgx.KgError, match="bad point value"):
        kgx.featurize_rows(kgx.make_positions([bad]), 9, 9)
    with pytest.raises(kgx.KgError, match="symmetry"):
        kgx.featurize_rows(kgx.make_positions([p]), 9, 9, symmetry=[8])
    with pytest.raises(kgx.KgError, match=r"\[1, 19\]"):
        kgx.featurize_rows(kgx.make_positions([p]), 20, 9)
