"""Featurizer test cases: the reference's fixture rows (tests/golden/featurize.npz, written by
tests/golden/gen_featurize.py from fixtures/upstream-v1.18.2/unit/oracle/nninputs_*.txt) and seeded random
positions; FNV-1a as the reference's fixtures fold floats (fixtures/upstream-v1.18.2/unit/oracle/nninputs.cpp:43-45);
and an independent flood-fill count of chain liberties."""

import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "featurize.npz")


def fnv1a(a) -> int:
    h = 0xCBF29CE484222325
    for b in np.ascontiguousarray(a, "<f4").tobytes():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def self_komi_from_g5(g5_bits, b_area):
    """The float32 s with fl(s / 20) == g5 (the fixture's g5 is fl(clip(self komi) / 20)): the clip bound when g5
    is at it, else, of the floats next to g5 * 20 that give g5, the one closest to a multiple of 0.05 (komi values
    and draw adjustments are such values)."""
    g5 = np.float32(struct.unpack("<f", struct.pack("<I", int(g5_bits)))[0])
    for bound in (np.float32(b_area + 20.0), np.float32(-b_area - 20.0)):
        if np.float32(bound / np.float32(20.0)) == g5:
            return float(bound)
    s0 = np.float32(g5 * np.float32(20.0))
    cands, up, down = [s0], s0, s0
    for _ in range(4):
        up = np.nextafter(up, np.float32(np.inf), dtype=np.float32)
        down = np.nextafter(down, np.float32(-np.inf), dtype=np.float32)
        cands += [up, down]
    ok = [c for c in cands if np.float32(c / np.float32(20.0)) == g5]
    assert ok, hex(int(g5_bits))
    return float(min(ok, key=lambda c: abs(float(c) * 20 - round(float(c) * 20))))


def self_komi_candidates(g5_bits, b_area):
    """Every float32 s within a few ulps of g5 * 20 with fl(clip(s) / 20) == g5 (a komi that is not a multiple of
    0.05 leaves a choice of two or three)."""
    g5 = np.float32(struct.unpack("<f", struct.pack("<I", int(g5_bits)))[0])
    out = [float(b) for b in (np.float32(b_area + 20.0), np.float32(-b_area - 20.0))
           if np.float32(b / np.float32(20.0)) == g5]
    s0 = np.float32(g5 * np.float32(20.0))
    cands, up, down = [s0], s0, s0
    for _ in range(6):
        up = np.nextafter(up, np.float32(np.inf), dtype=np.float32)
        down = np.nextafter(down, np.float32(-np.inf), dtype=np.float32)
        cands += [up, down]
    return out + [float(c) for c in cands if np.float32(c / np.float32(20.0)) == g5]


def fixture():
    return np.load(GOLDEN)


def fixture_positions():
    """[(position dict, (pos id, eval idx, symmetry, nn_x, nn_y), global bits, hashes)] for the 57 dumped rows."""
    g = fixture()
    out = []
    for i in range(len(g["meta"])):
        p = dict(meta=g["meta"][i], color=g["color"][i], marks=g["marks"][i], area=g["area"][i], enc=g["enc"][i],
                 moves=g["moves"][i], self_komi=float(g["self_komi_bits"][i:i + 1].view(np.float32)[0]),
                 pda=float(g["pda"][i]))
        out.append((p, tuple(int(v) for v in g["layout"][i]), g["glob_bits"][i], [int(v) for v in g["hashes"][i]]))
    return out


def random_position(rng, xs=None, ys=None):
    xs = int(rng.integers(1, 20)) if xs is None else xs
    ys = int(rng.integers(1, 20)) if ys is None else ys
    n = xs * ys
    pla = int(rng.integers(1, 3))
    fill = rng.uniform(0.2, 0.8)
    color = np.zeros(361, np.uint8)
    color[:n] = np.where(rng.random(n) < fill, rng.integers(1, 3, n), 0)
    marks = np.zeros(361, np.uint8)
    marks[:n] = rng.integers(0, 64, n) * (rng.random(n) < 0.15)
    area = np.zeros(361, np.uint8)
    area[:n] = rng.integers(0, 3, n)
    enc = np.zeros(361, np.uint8)
    enc[:n] = rng.integers(0, 3, n)
    empties = np.flatnonzero(color[:n] == 0)
    ko_loc = int(rng.choice(empties)) if len(empties) and rng.random() < 0.5 else -1
    encore = int(rng.integers(0, 3))
    nm = int(rng.integers(0, 6))
    moves = np.full(10, -2, np.int32)
    moves[1::2] = 0
    for k in range(nm):
        r = rng.random()
        moves[2 * k] = -1 if r < 0.15 else -2 if r < 0.2 else int(rng.integers(0, n))
        # mostly alternating opp, pla, ...; sometimes the same player twice (the history then stops there)
        want = 3 - pla if k % 2 == 0 else pla
        moves[2 * k + 1] = want if rng.random() < 0.85 else 3 - want
    meta = np.array([xs, ys, pla, ko_loc, encore, int(rng.integers(0, 4)), int(rng.integers(0, 2)),
                     int(rng.integers(0, 3)), int(rng.integers(0, 2)), int(rng.integers(0, 2)),
                     int(rng.integers(0, 2)), int(rng.integers(0, 6)), nm], np.int32)
    r = rng.random()
    komi = (float(rng.integers(-800, 800)) / 2 if r < 0.5 else float(rng.uniform(-450, 450)) if r < 0.9
            else float(np.float32(rng.choice([1, -1]) * (n + 20 + rng.uniform(-1, 1)))))
    pda = 0.0 if rng.random() < 0.6 else float(rng.uniform(-3, 3))
    return dict(meta=meta, color=color, marks=marks, area=area, enc=enc, moves=moves,
                self_komi=float(np.float32(komi)), pda=pda)


def liberties_bruteforce(color, xs, ys):
    """Per point: the number of distinct empty points next to the stone's chain (0 for empty points)."""
    n = xs * ys
    out = np.zeros(n, np.int32)
    for p in range(n):
        if color[p] == 0:
            continue
        chain, todo, libs = {p}, [p], set()
        while todo:
            q = todo.pop()
            x, y = q % xs, q // xs
            for nx, ny in ((x - 1, y), (x + 1, y), (x, y - 1), (x, y + 1)):
                if 0 <= nx < xs and 0 <= ny < ys:
                    r = nx + ny * xs
                    if color[r] == 0:
                        libs.add(r)
                    elif color[r] == color[p] and r not in chain:
                        chain.add(r)
                        todo.append(r)
        out[p] = len(libs)
    return out
