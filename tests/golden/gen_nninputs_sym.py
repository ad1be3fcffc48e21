"""Writes tests/golden/nninputs_sym.npz from the reference's NN-input oracle fixtures.

Source (data files of the reference's own test suite, read as text):
  fixtures/upstream-v1.18.2/unit/oracle/nninputs_positions.txt  (eval lines: symmetry, nnXLen, nnYLen)
  fixtures/upstream-v1.18.2/unit/oracle/nninputs_expected.txt   (res lines: FNV-1a hashes; dump lines: every
                                                                 nonzero NCHW input-row entry of some evals)
Their format is documented in fixtures/upstream-v1.18.2/unit/oracle/nninputs.cpp:43-64. For each eval with a
dump line this keeps the input row (sparse: index and f32 bits) and three hashes of the res line:
  fnv_nchw     FNV-1a of the 22 * nnYLen * nnXLen row floats
  fnv_sym_in   FNV-1a of copyInputsWithSymmetry(row, 1, nnYLen, nnXLen, 22, NCHW, sym)
  fnv_sym_out  FNV-1a of copyOutputsWithSymmetry(channel-0 plane, 1, nnYLen, nnXLen, sym)
with sym = the eval's symmetry if >= 0, else 0.

Run: python tests/golden/gen_nninputs_sym.py  (REFERENCE env var, default /root/reference)
"""

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    ref = os.environ.get("REFERENCE", "/root/reference")
    d = os.path.join(ref, "fixtures", "upstream-v1.18.2", "unit", "oracle")
    evals = {}
    for line in open(os.path.join(d, "nninputs_positions.txt")):
        if line.startswith("eval "):
            f = line.split()
            evals[(int(f[1]), int(f[2]))] = (int(f[10]), int(f[13]), int(f[14]))  # symmetry, nnXLen, nnYLen
    res, dumps = {}, {}
    for line in open(os.path.join(d, "nninputs_expected.txt")):
        f = line.split()
        if f and f[0] == "res":
            key = (int(f[1]), int(f[2]))
            res[key] = (int(f[5], 16), int(f[-3], 16), int(f[-1], 16))
        elif f and f[0] == "dump":
            key, n = (int(f[1]), int(f[2])), int(f[3])
            e = f[4:]
            assert len(e) == 3 * n
            dumps[key] = [(int(e[3 * i]), int(e[3 * i + 1]), int(e[3 * i + 2], 16)) for i in range(n)]
    keys = sorted(dumps)
    meta, hashes, nz_case, nz_index, nz_bits = [], [], [], [], []
    for ci, key in enumerate(keys):
        sym, nx, ny = evals[key]
        meta.append((key[0], key[1], sym, nx, ny))
        hashes.append(res[key])
        for c, pos, bits in dumps[key]:
            nz_case.append(ci)
            nz_index.append(c * nx * ny + pos)
            nz_bits.append(bits)
    np.savez_compressed(os.path.join(HERE, "nninputs_sym.npz"),
                        meta=np.array(meta, np.int32),            # pos id, eval idx, symmetry, nnXLen, nnYLen
                        hashes=np.array(hashes, np.uint64),       # fnv_nchw, fnv_sym_in, fnv_sym_out
                        nz_case=np.array(nz_case, np.int32), nz_index=np.array(nz_index, np.int32),
                        nz_bits=np.array(nz_bits, np.uint32))
    print(f"wrote nninputs_sym.npz: {len(keys)} evals, {len(nz_bits)} nonzero entries")


if __name__ == "__main__":
    main()
