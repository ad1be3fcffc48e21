"""Writes tests/golden/modelversion_desc.json from the reference's fixture
fixtures/upstream-v1.18.2/unit/oracle/modelversion_desc.txt (KataGo v1.18.2's own NNModelVersion outputs, written by
modelversion_desc.cpp beside it): the per-version input feature counts (lines "V <fn> <arg> <value>" or
"V <fn> <arg> ERR <text>") and the ModelPostProcessParams defaults (lines "P <field> <f64 bits>"). The rules lines
(R) belong to the engine, not to the forward pass, and are left out.

Run: python tests/golden/gen_modelversion.py (reads the reference checkout at $REFERENCE, default /root/reference).
"""

import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    ref = os.environ.get("REFERENCE", "/root/reference")
    src = os.path.join(ref, "fixtures", "upstream-v1.18.2", "unit", "oracle", "modelversion_desc.txt")
    vals, post = [], {}
    for line in open(src):
        f = line.split()
        if not f:
            continue
        if f[0] == "V":
            fn, arg = f[1], int(f[2])
            if f[3] == "ERR":
                vals.append({"fn": fn, "arg": arg, "err": " ".join(f[4:])})
            else:
                vals.append({"fn": fn, "arg": arg, "value": int(f[3])})
        elif f[0] == "P":
            bits = int(f[2], 16)
            post[f[1]] = struct.unpack("<d", struct.pack("<Q", bits))[0] if len(f[2]) == 16 else \
                struct.unpack("<f", struct.pack("<I", bits))[0]
    out = os.path.join(HERE, "modelversion_desc.json")
    with open(out, "w") as fh:
        json.dump({"source": "fixtures/upstream-v1.18.2/unit/oracle/modelversion_desc.txt", "V": vals, "P": post},
                  fh, indent=0)
    print("wrote", out, len(vals), "V lines,", len(post), "P lines")


if __name__ == "__main__":
    main()
