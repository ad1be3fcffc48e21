"""Writes tests/golden/nneval_skipnn.npz from the reference's fixture
fixtures/upstream-v1.18.2/unit/oracle/nneval_skipnn.txt (KataGo v1.18.2's NNEvaluator with debugSkipNeuralNet,
written by nneval_skipnn.cpp beside it; replayed by crates/katago-core/tests/nneval_skipnn.rs).

In that mode the evaluator's serve task fills each row's raw outputs from its own random stream
(crates/katago-core/src/neuralnet/nneval.rs:863-935) and evaluate() then runs the ordinary post-processing
(nneval.rs:1197-1500) at the default model version 17. The fixture prints the op stream (E evaluator, P position,
V/W/A evaluations, K server respawn, S end) and the results: an R line per evaluation (hashes, the nine value
fields, policy FNV, owner FNV) and, for the first six V/A evaluations of each evaluator, a D line with every policy
probability and ownership value as float bits.

This script regenerates those raw outputs: the serve task's Rand (seeded "<seed>:NNEvalServerThread:<n>", n
counting spawns) restated below from its published algorithm (core/rand.rs: MD5 + SHA-256 seeding,
xorshift1024* plus PCG32, polar Box-Muller gaussians), checked against the known-answer sequences of the
reference's own XorShift1024Mult::test and PCG32::test. An evaluation draws new values unless the NN cache
returns an earlier result: the cache exists when the E line's cache size is >= 0, is read unless skipCache,
and holds a result per nnHash (the R line's hashes); a cached result without an owner map does not serve a
request that needs one (nneval.rs:1127-1140). The replay of an evaluator stops at its first A line
(averageMultipleSymmetries draws for symmetries the fixture does not print), so only evaluations before it are
kept, and only those with a D line that drew their own values (not cache hits, whose output repeats an earlier
one, nor the owner-map re-evaluations, which keep the cached fields).

For each kept evaluation the npz holds: the raw values in this repository's row layout (19x19 positions), the
legality mask (the D line's -1 entries: history.is_legal plus the dagger ban, which need the rules engine), the
parameters, and the expected policy, ownership and value fields as float bits. Legal move masks are thereby data
from the fixture, not computed here.

Run: python tests/golden/gen_nneval_skipnn.py (reads the reference checkout at $REFERENCE, default /root/reference).
"""

import hashlib
import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


class XorShift1024Mult:
    """xorshift1024* (http://xoroshiro.di.unimi.it/), 16 words of state, upper 32 bits of the product."""

    def __init__(self, words):
        self.a = list(words)
        self.i = 0

    def next_uint(self):
        a0 = self.a[self.i]
        self.i = (self.i + 1) & 15
        a1 = self.a[self.i]
        a1 ^= (a1 << 31) & M64
        a1 ^= a1 >> 11
        a0 ^= a0 >> 30
        self.a[self.i] = a0 ^ a1
        return ((self.a[self.i] * 1181783497276652981) & M64) >> 32


class PCG32:
    """PCG32 (http://www.pcg-random.org/): 64-bit LCG state, xorshift-rotate output."""

    def __init__(self, state):
        self.s = state & M64

    def next_uint(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & M64
        x = (((self.s >> 18) ^ self.s) >> 27) & 0xFFFFFFFF
        rot = self.s >> 59
        return x if rot == 0 else ((x >> rot) | (x << (32 - rot))) & 0xFFFFFFFF


class Rand:
    """KataGo's Rand: next_uint = PCG32 + xorshift1024* (mod 2^32), seeded from a string through MD5 and SHA-256."""

    def __init__(self, seed):
        h0 = struct.unpack("<I", hashlib.md5(seed.encode()).digest()[:4])[0]
        s = "|" + str(h0) + "|" + seed
        state = {"counter": 0, "idx": 4, "hash": [0, 0, 0, 0]}

        def nonzero():
            while True:
                if state["idx"] >= 4:
                    d = hashlib.sha256((str(state["counter"]) + s).encode()).digest()
                    state["counter"] += 37
                    state["hash"] = list(struct.unpack(">4Q", d))
                    state["idx"] = 0
                v = state["hash"][state["idx"]]
                state["idx"] += 1
                if v != 0:
                    return v

        words = [nonzero() for _ in range(16)]
        self.xorm = XorShift1024Mult(words)
        self.pcg = PCG32(nonzero())
        self.stored = None

    def next_uint(self):
        return (self.pcg.next_uint() + self.xorm.next_uint()) & 0xFFFFFFFF

    def next_double(self):
        while True:
            lower = self.next_uint()
            upper = self.next_uint()
            x = (((upper << 32) | lower) & ((1 << 53) - 1)) / float(1 << 53)
            if 0.0 <= x < 1.0:
                return x

    def next_gaussian(self):
        if self.stored is not None:
            g, self.stored = self.stored, None
            return g
        while True:
            v1 = self.next_double() * 2.0 - 1.0
            v2 = self.next_double() * 2.0 - 1.0
            s = v1 * v1 + v2 * v2
            if not (s >= 1.0 or s == 0.0):
                break
        mult = math.sqrt(-2.0 * math.log(s) / s)
        self.stored = v2 * mult
        return v1 * mult


# Known answers of the reference's own generator self-tests (core/rand.rs, XorShift1024Mult::test and PCG32::test).
XORM_INIT = [15148282349006049087, 3601266951833665894, 16929445066801446424, 13475938501103070154,
             15713138009143754412, 4148159782736716337, 16035594834001032141, 5555591070439871209,
             4101130512537511022, 12821547636792886909, 9050874162294428797, 6187760405891629771,
             10053646276519763308, 2219782655280501359, 3719698449347562208, 5421263376768154227]
XORM_EXPECTED = [0x749746d1, 0x9242ca14, 0x98db98a1, 0x1348e491, 0xde60e668, 0x77e37a69, 0xeb51a9d3, 0xd44b4727,
                 0x341895b0, 0xc7b1b3f4, 0xe7ef0529, 0x8e72ea7e, 0x5855da19, 0xfffcd2b2, 0xa684e430, 0xb76a7e0d,
                 0x5af3820e, 0x320b0699, 0xdbb85ee0, 0xc1dcd25c, 0x4b395e3e, 0x4007756f, 0x76a0c667, 0xaa6041f6,
                 0x756f94bb, 0x39527d1b, 0x6e1232ef, 0xb3027668, 0x776ea832, 0x35a0ed1b, 0x1f2f0268, 0xadd59669]
PCG_EXPECTED = [0xb3766cbd, 0x65fdd305, 0x2a3b9b9c, 0x09a2dee9, 0x1a86aabc, 0x36a98234, 0x82e6e2b4, 0x10c077e5,
                0x29755fc7, 0xf7fa7b5c, 0x1cb7ae7d, 0xcce0e3d9, 0x065ec08b, 0x505d1cdb, 0x8b778f3c, 0xdb72f217]


def check_generators():
    x = XorShift1024Mult(XORM_INIT)
    assert [x.next_uint() for _ in range(32)] == XORM_EXPECTED, "xorshift1024* known answers"
    p = PCG32(123)
    assert [p.next_uint() for _ in range(16)] == PCG_EXPECTED, "PCG32 known answers"


def f32(v):
    return float(np.float32(v))


def bits_f32(h):
    return struct.unpack("<f", struct.pack("<I", int(h, 16)))[0]


def bits_f64(h):
    return struct.unpack("<d", struct.pack("<Q", int(h, 16)))[0]


def replay(path):
    lines = [ln.rstrip("\n") for ln in open(path)]
    cases = []
    k = 0
    cfg = None
    while k < len(lines):
        f = lines[k].split(" ")
        op = f[0]
        if op == "E":
            cfg = {"nx": int(f[1]), "ny": int(f[2]), "cache": {} if int(f[3]) >= 0 else None, "seed": f[4],
                   "spawned": 1, "evals": 0, "live": True}
            cfg["rand"] = Rand(cfg["seed"] + ":NNEvalServerThread:0")
            pos = None
        elif op == "P":
            bx, by = int(f[1]), int(f[2])
            ko, scoring = int(f[3]), int(f[4])
            pla, n = int(f[11]), int(f[12])
            for m in range(n):
                pla = 3 - int(f[14 + 2 * m])  # presumed next player: the opponent of each move's player
            pos = {"bx": bx, "by": by, "next": pla, "no_result": ko == 0 or scoring == 1}
        elif op == "K":
            cfg["rand"] = Rand(cfg["seed"] + ":NNEvalServerThread:" + str(cfg["spawned"]))
            cfg["spawned"] += 1
        elif op in ("V", "W", "A"):
            r = lines[k + 1].split(" ")
            assert r[0] == "R", lines[k + 1][:40]
            d = lines[k + 2].split(" ") if k + 2 < len(lines) and lines[k + 2].startswith("D ") else None
            temperature = bits_f32(f[5])
            passing = f[3] == "1"
            optimism = bits_f64(f[8])
            skip_cache, owner = f[10] == "1", f[11] == "1"
            nn_hash = (r[1], r[2])
            if op == "A":
                cfg["live"] = False
                cfg["evals"] += 1
            elif cfg["live"]:
                cache = cfg["cache"]
                hit = partial = False
                if cache is not None and not skip_cache and nn_hash in cache:
                    if owner and not cache[nn_hash]:
                        partial = True
                    else:
                        hit = True
                raw = None
                if not hit:
                    rnd, bx, by, nx = cfg["rand"], pos["bx"], pos["by"], cfg["nx"]
                    pol = np.zeros(362, np.float32)
                    for y in range(by):
                        for x in range(bx):
                            pol[y * 19 + x] = f32(rnd.next_gaussian())
                    pol[361] = f32(rnd.next_gaussian())
                    own = np.zeros(361, np.float32)
                    if owner:
                        for y in range(by):
                            for x in range(bx):
                                own[y * 19 + x] = np.float32(f32(rnd.next_gaussian())) * np.float32(0.20)
                    win = f32(0.0 + rnd.next_gaussian() * 0.20)
                    loss = f32(0.0 + rnd.next_gaussian() * 0.20)
                    mean = f32(0.0 + rnd.next_gaussian() * 0.20)
                    mean_sq = f32(0.0 + rnd.next_gaussian() * 0.20)
                    nores = f32(0.0 + rnd.next_gaussian() * 0.20)
                    var = f32(0.5 * bx * by)
                    raw = {"policy": pol, "owner": own, "value": np.array([win, loss, nores], np.float32),
                           "score": np.array([mean, mean_sq, mean, var, 0.0, 0.0], np.float32)}
                if cache is not None and not hit:
                    cache[nn_hash] = owner  # every evaluation that ran stores its result (nneval.rs:1506-1511)
                if op == "V":
                    cfg["evals"] += 1
                if d is not None and raw is not None and not partial:
                    nx, ny = cfg["nx"], cfg["ny"]
                    bar = d.index("|")
                    dp = [int(h, 16) for h in d[1:bar]]
                    do = [int(h, 16) for h in d[bar + 1:]]
                    assert len(dp) == nx * ny + 1 and len(do) == (nx * ny if owner else 0)
                    exp_pol = np.full(362, 0xBF800000, np.uint32)
                    exp_own = np.zeros(361, np.uint32)
                    for y in range(ny):
                        for x in range(nx):
                            exp_pol[y * 19 + x] = dp[y * nx + x]
                            if owner:
                                exp_own[y * 19 + x] = do[y * nx + x]
                    exp_pol[361] = dp[nx * ny]
                    legal = (exp_pol != 0xBF800000).astype(np.uint8)
                    fields = np.array([int(h, 16) for h in r[3:12]], np.uint32)
                    cases.append({"line": k + 1, "bx": pos["bx"], "by": pos["by"], "white": pos["next"] == 2,
                                  "no_result": pos["no_result"], "temperature": temperature, "passing": passing,
                                  "optimism": optimism, "owner": owner, "legal": legal, "raw": raw,
                                  "exp_policy": exp_pol, "exp_owner": exp_own, "exp_fields": fields})
        k += 1
    return cases


def main():
    check_generators()
    ref = os.environ.get("REFERENCE", "/root/reference")
    src = os.path.join(ref, "fixtures", "upstream-v1.18.2", "unit", "oracle", "nneval_skipnn.txt")
    cases = replay(src)
    n = len(cases)
    out = os.path.join(HERE, "nneval_skipnn.npz")
    np.savez_compressed(
        out,
        line=np.array([c["line"] for c in cases], np.int32),
        board=np.array([[c["bx"], c["by"]] for c in cases], np.int32),
        white=np.array([c["white"] for c in cases], np.uint8),
        no_result=np.array([c["no_result"] for c in cases], np.uint8),
        temperature=np.array([c["temperature"] for c in cases], np.float32),
        passing=np.array([c["passing"] for c in cases], np.uint8),
        optimism=np.array([c["optimism"] for c in cases], np.float64),
        owner=np.array([c["owner"] for c in cases], np.uint8),
        legal=np.stack([c["legal"] for c in cases]),
        raw_policy=np.stack([c["raw"]["policy"] for c in cases]),
        raw_owner=np.stack([c["raw"]["owner"] for c in cases]),
        raw_value=np.stack([c["raw"]["value"] for c in cases]),
        raw_score=np.stack([c["raw"]["score"] for c in cases]),
        exp_policy=np.stack([c["exp_policy"] for c in cases]),
        exp_owner=np.stack([c["exp_owner"] for c in cases]),
        exp_fields=np.stack([c["exp_fields"] for c in cases]),
    )
    print("wrote", out, n, "evaluations (lines", [c["line"] for c in cases], ")")


if __name__ == "__main__":
    main()
