"""Writes tests/golden/featurize.npz from the reference's NN-input oracle fixtures.

Source (data files of the reference's own test suite, read as text):
  fixtures/upstream-v1.18.2/unit/oracle/nninputs_positions.txt  (pos lines: board size and rules; eval lines:
                                                                 next player, playout doubling advantage,
                                                                 symmetry, nnXLen, nnYLen)
  fixtures/upstream-v1.18.2/unit/oracle/nninputs_expected.txt   (res lines: FNV-1a hashes of fillRowV7's rows and
                                                                 the 19 global features; dump lines: every
                                                                 nonzero NCHW spatial entry of some evals)
Their format is documented in fixtures/upstream-v1.18.2/unit/oracle/nninputs.cpp:23-64.

Two sets of cases:
- "rows": every eval with a dump line. The featurizer's inputs are read back from the dump and the res line:
  the stones from features 1/2 (and the next player), the superko / ko-recapture marks from features 6/7, the
  ladder marks from 14-17, the area colours from 18/19, the second-encore colours from 20/21, the move history
  from features 9-13 and the pass flags g0-g4, the encore phase from g12/g13, pass_would_end_phase from g14,
  hist.has_button from g17 (the button is history state: it is gone once a player has taken it), and
  the self komi as the float s with fl(s / 20) = g5 (or the clip bound). The features the featurizer computes
  itself (on-board, liberties 1/2/3, the parity wave g18, every layout and symmetry) are then checked against the
  fixture: bit for bit against the dump, and through the reference's FNV-1a hashes of the whole row (NCHW and
  NHWC, before and after the eval's symmetry).
- "globals": every res line (4035 evals): board size, scoring rule, encore phase, g5 and g18, for the komi clip,
  scaling and parity wave over the whole fixture.

Run: python tests/golden/gen_featurize.py  (REFERENCE env var, default /root/reference)
"""

import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from featurize_cases import self_komi_from_g5  # noqa: E402


def main():
    ref = os.environ.get("REFERENCE", "/root/reference")
    d = os.path.join(ref, "fixtures", "upstream-v1.18.2", "unit", "oracle")
    poss, evals = {}, {}
    for line in open(os.path.join(d, "nninputs_positions.txt")):
        f = line.split()
        if not f:
            continue
        if f[0] == "pos":
            # pos id xSize ySize koRule scoringRule taxRule suicide button whbRule friendlyPassOk komi ...
            poss[int(f[1])] = dict(xs=int(f[2]), ys=int(f[3]), ko=int(f[4]), scoring=int(f[5]), tax=int(f[6]),
                                   suicide=int(f[7]), button=int(f[8]))
        elif f[0] == "eval":
            # eval pos idx nextPla drawEquiv cpr passHacks pda temp dagger sym optimism maxHist nnX nnY
            evals[(int(f[1]), int(f[2]))] = dict(pla=int(f[3]), pda=struct.unpack("<d", bytes.fromhex(f[7])[::-1])[0],
                                                 sym=int(f[10]), nnx=int(f[13]), nny=int(f[14]))
    res, dumps = {}, {}
    for line in open(os.path.join(d, "nninputs_expected.txt")):
        f = line.split()
        if not f:
            continue
        if f[0] == "res":
            key = (int(f[1]), int(f[2]))
            res[key] = dict(fnv_nchw=int(f[5], 16), fnv_nhwc=int(f[6], 16),
                            glob=[int(v, 16) for v in f[7:26]],
                            fnv_sym_nchw=int(f[26], 16), fnv_sym_nhwc=int(f[27], 16))
        elif f[0] == "dump":
            key, n = (int(f[1]), int(f[2])), int(f[3])
            e = f[4:]
            assert len(e) == 3 * n
            dumps[key] = [(int(e[3 * i]), int(e[3 * i + 1]), int(e[3 * i + 2], 16)) for i in range(n)]

    # rows
    meta, color, marks, area, enc, moves, komi, pda, layout, glob, hashes = ([] for _ in range(11))
    for key in sorted(dumps):
        p, e, r = poss[key[0]], evals[key], res[key]
        xs, ys, nnx, pla = p["xs"], p["ys"], e["nnx"], e["pla"]
        opp = 3 - pla
        feat = {}
        for c, pos, bits in dumps[key]:
            assert bits == 0x3F800000, "spatial features are 0/1"
            feat.setdefault(c, set()).add(pos)
        g = r["glob"]
        encore = 2 if g[13] else 1 if g[12] else 0
        col, mk, ar, en = (np.zeros(361, np.uint8) for _ in range(4))
        for y in range(ys):
            for x in range(xs):
                pos, loc = y * nnx + x, x + y * xs
                assert pos in feat.get(0, ()), "on-board plane"
                col[loc] = pla if pos in feat.get(1, ()) else opp if pos in feat.get(2, ()) else 0
                mk[loc] = (pos in feat.get(6, ())) | ((pos in feat.get(7, ())) << 1)
                for b in range(4):
                    mk[loc] |= (pos in feat.get(14 + b, ())) << (2 + b)
                ar[loc] = pla if pos in feat.get(18, ()) else opp if pos in feat.get(19, ()) else 0
                en[loc] = pla if pos in feat.get(20, ()) else opp if pos in feat.get(21, ()) else 0
        mv = []
        for k in range(5):
            locs = feat.get(9 + k, set())
            assert len(locs) <= 1
            if g[k]:
                mv.append((-1, opp if k % 2 == 0 else pla))
            elif locs:
                pos = next(iter(locs))
                mv.append(((pos // nnx) * xs + pos % nnx, opp if k % 2 == 0 else pla))
            else:
                break
        turns = len(mv)
        mv += [(-2, 0)] * (5 - len(mv))
        s = self_komi_from_g5(g[5], xs * ys)
        meta.append([xs, ys, pla, -1, encore, p["ko"], p["scoring"], p["tax"], p["suicide"], 1 if g[17] else 0,
                     1 if g[14] else 0, turns, turns])
        color.append(col), marks.append(mk), area.append(ar), enc.append(en)
        moves.append(np.array(mv, np.int32).reshape(-1))
        komi.append(np.float32(s).view(np.uint32))
        pda.append(e["pda"])
        layout.append([key[0], key[1], e["sym"], e["nnx"], e["nny"]])
        glob.append(g)
        hashes.append([r["fnv_nchw"], r["fnv_nhwc"], r["fnv_sym_nchw"], r["fnv_sym_nhwc"]])

    # globals over every res line
    gl = []
    for key in sorted(res):
        p, r = poss[key[0]], res[key]
        g = r["glob"]
        encore = 2 if g[13] else 1 if g[12] else 0
        gl.append([p["xs"], p["ys"], p["scoring"], encore, g[5], g[18]])

    np.savez_compressed(os.path.join(HERE, "featurize.npz"),
                        meta=np.array(meta, np.int32), color=np.array(color), marks=np.array(marks),
                        area=np.array(area), enc=np.array(enc), moves=np.array(moves, np.int32),
                        self_komi_bits=np.array(komi, np.uint32), pda=np.array(pda, np.float64),
                        layout=np.array(layout, np.int32), glob_bits=np.array(glob, np.uint32),
                        hashes=np.array(hashes, np.uint64), all_glob=np.array(gl, np.int64))
    print(f"wrote featurize.npz: {len(meta)} rows, {len(gl)} global records")


if __name__ == "__main__":
    main()
