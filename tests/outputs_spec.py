"""The NNOutput fields of one readback row as copy_outputs (crates/katago-nn-burn/src/backend.rs:622-731) defines
them, written out branch by branch, for sentinel tests of the library's and the oracle's unpacking."""

import numpy as np

HW = 361


def score_channels(v):
    """The value head's score channels by model version (bin2onnx.py:849-856)."""
    return 6 if v >= 9 else 4 if v >= 8 else 2 if v >= 4 else 1


def sentinel_row(P, S, base=1000.0):
    """A raw row whose every slot holds a distinct, exactly representable value."""
    return (base + np.arange(P * (HW + 1) + 3 + S + HW)).astype(np.float32)


def expected(raw, P, S, v, optimism):
    """(policy [362] before symmetry, 9 scalar fields, ownership [361] before symmetry)."""
    f = np.float32
    pol = raw[:P * (HW + 1)]
    o = f(optimism)
    if P == 2 or (P == 4 and v >= 16):  # backend.rs:661: the optimistic channel 1 is mixed into channel 0
        policy = (pol[:HW] + (pol[HW + 1:HW + 1 + HW] - pol[:HW]) * o).astype(np.float32)
        pas = f(pol[HW] + (pol[(HW + 1) + HW] - pol[HW]) * o)  # pass logits at c * 362 + 361
    else:  # backend.rs:669-672: channel 0 only
        policy = pol[:HW].copy()
        pas = pol[HW]
    val = raw[P * (HW + 1):P * (HW + 1) + 3]                      # backend.rs:677-680
    sc = raw[P * (HW + 1) + 3:P * (HW + 1) + 3 + S]
    own = raw[P * (HW + 1) + 3 + S:]
    if v >= 9:    # backend.rs:688-696
        score = [sc[0], sc[1], sc[2], sc[3], sc[4], sc[5]]
    elif v >= 8:  # backend.rs:697-705
        score = [sc[0], sc[1], sc[2], sc[3], 0.0, 0.0]
    elif v >= 4:  # backend.rs:706-714
        score = [sc[0], sc[1], sc[0], 0.0, 0.0, 0.0]
    else:         # backend.rs:715-724: no second moment in version 3 nets, the mean squared stands in
        score = [sc[0], f(sc[0] * sc[0]), sc[0], 0.0, 0.0, 0.0]
    fields = np.array([val[0], val[1], val[2]] + score, np.float32)
    return np.append(policy, pas).astype(np.float32), fields, own.copy()


FIELDS = ("white_win_prob", "white_loss_prob", "white_no_result_prob", "white_score_mean", "white_score_mean_sq",
          "white_lead", "var_time_left", "shortterm_winloss_error", "shortterm_score_error")

# (model version, policy channels): every version branch of the score unpacking, and every branch of the policy
# (P = 1; P = 2; P = 4 from version 16, and P = 4 before it, which reads channel 0 only).
CASES = [(17, 4), (16, 4), (15, 4), (15, 2), (12, 2), (11, 1), (9, 1), (8, 1), (7, 1), (5, 1), (4, 1), (3, 1)]
OPTIMISMS = (0.0, 1.0, 0.25)
