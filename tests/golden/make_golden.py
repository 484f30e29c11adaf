"""Writes tests/golden/dgda_golden.json: DGDA cases whose outputs were worked
out by hand (exact binary fractions), independent of the oracle code.

Case "hand_2tok" (dk = dv = 2, one batch and head), per token t:
  S' = diag(alpha_t) S;  pred = (b_t*k_t)^T S';  delta = w_t*v_t - pred
  S  = S' + k_t delta^T;  o_t = S^T q_t
  t=0: S0 = [[1,2],[3,4]], alpha=[.5,1] -> S' = [[.5,1],[3,4]]; k=[1,0], b=[1,1]
       pred = [.5,1]; w*v = [10,20]; delta = [9.5,19]; S = [[10,20],[3,4]];
       q = [1,1] -> o = [13,24]
  t=1: alpha=[1,.5] -> S' = [[10,20],[1.5,2]]; k=[0,1], b=[.5,1] -> bk=[0,1]
       pred = [1.5,2]; w=[1,.5], v=[2,4] -> w*v=[2,2]; delta=[.5,0]
       S = [[10,20],[2,2]]; q=[0,2] -> o = [4,4]
Case "zero_state_one_tok": S0 = 0, so S = k (w*v)^T and o = (q.k) w*v:
  k=[0.6,0.8] (unit), w*v = [1,-2,0.5], q=[1,2] -> q.k = 2.2
  S = [[.6,-1.2,.3],[.8,-1.6,.4]], o = [2.2,-4.4,1.1]
"""
import json
import os

cases = [
    {
        "name": "hand_2tok",
        "inputs": {
            "q": [[[[1, 1], [0, 2]]]],
            "k": [[[[1, 0], [0, 1]]]],
            "v": [[[[10, 20], [2, 4]]]],
            "alpha": [[[[0.5, 1], [1, 0.5]]]],
            "b": [[[[1, 1], [0.5, 1]]]],
            "w": [[[[1, 1], [1, 0.5]]]],
            "initial_state": [[[[1, 2], [3, 4]]]],
        },
        "out": [[[[13, 24], [4, 4]]]],
        "state": [[[[10, 20], [2, 2]]]],
    },
    {
        "name": "zero_state_one_tok",
        "inputs": {
            "q": [[[[1, 2]]]],
            "k": [[[[0.6, 0.8]]]],
            "v": [[[[2, -4, 1]]]],
            "alpha": [[[[0.3, 0.7]]]],
            "b": [[[[0.9, 0.1]]]],
            "w": [[[[0.5, 0.5, 0.5]]]],
        },
        "out": [[[[2.2, -4.4, 1.1]]]],
        "state": [[[[0.6, -1.2, 0.3], [0.8, -1.6, 0.4]]]],
    },
]

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dgda_golden.json")
    with open(out, "w") as fh:
        json.dump(cases, fh, indent=1)
    print(out)
