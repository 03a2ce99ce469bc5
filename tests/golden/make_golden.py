"""Writes the known-answer fixtures of tests/golden/.

The inputs are the literals of the reference's own known-answer tests; the
expected outputs are derived by hand below (each line says how), not by
running any implementation:

* pack_kat.json    — reference tests/test_packing.py:14-47 (4 tokens, d=2,
  top-2 over 3 experts, offsets [0,4,6,8]). The reference test checks only
  segment membership and row identity (:65-76); the expected arrays here
  add the canonical in-segment order (stable by flat assignment index, the
  order of the reference torch backend, src/model/torch_backend.py:58-66),
  plus a hand-computed pack backward on the same routing.
* combine_kat.json — reference tests/test_combine.py:20-42 (top-1
  permutation) and :54-90 (top-2, literal weights), with the sums done by
  hand in decimal.

Run: python tests/golden/make_golden.py
"""

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent


def pack_kat():
    X = [[0.1, 0.2], [0.3, 0.4], [0.5, 0.6], [0.8, 0.8]]
    topk = [[0, 1], [0, 2], [1, 0], [0, 2]]
    w = [[0.7, 0.3], [0.6, 0.4], [0.9, 0.1], [0.1, 0.9]]
    cursor = [0, 4, 6, 8]
    # Flat assignments f = 2t + j with experts [0,1,0,2,1,0,0,2]:
    #   expert 0 <- f 0,2,5,6 (tokens 0,1,2,3) -> slots 0..3
    #   expert 1 <- f 1,4     (tokens 0,2)     -> slots 4,5
    #   expert 2 <- f 3,7     (tokens 1,3)     -> slots 6,7
    token_id = [0, 1, 2, 3, 0, 2, 1, 3]
    expert = [0, 0, 0, 0, 1, 1, 2, 2]
    packed_w = [0.7, 0.6, 0.1, 0.1, 0.3, 0.9, 0.4, 0.9]
    inv = [[0, 4], [1, 6], [5, 2], [3, 7]]  # slot of (t, j)
    packed_X = [X[t] for t in token_id]
    counts = [4, 2, 2]
    cursor_after = [4, 6, 8, 8]
    # Pack backward with packed-row grads dpX[p] = [p, 10p] and dpw[p] = p/2:
    # dX[t] = sum of its rows: t0 rows 0,4 -> [4,40]; t1 rows 1,6 -> [7,70];
    # t2 rows 2,5 -> [7,70]; t3 rows 3,7 -> [10,100].
    # dw[t, j] = dpw[inv[t, j]].
    dpX = [[p, 10 * p] for p in range(8)]
    dpw = [p / 2 for p in range(8)]
    dX = [[4, 40], [7, 70], [7, 70], [10, 100]]
    dw = [[0.0, 2.0], [0.5, 3.0], [2.5, 1.0], [1.5, 3.5]]
    return {
        "source": "reference tests/test_packing.py:14-76",
        "inputs": {"X": X, "topk_experts": topk, "topk_weights": w, "expert_offset_cpy": cursor},
        "expected": {
            "counts": counts,
            "packed_tokenId": token_id,
            "packed_expert": expert,
            "packed_topk_weights": packed_w,
            "packed_X": packed_X,
            "inv": inv,
            "cursor_after": cursor_after,
        },
        "backward": {"packed_X_grad": dpX, "packed_topk_weights_grad": dpw, "X_grad": dX,
                     "topk_weights_grad": dw},
    }


def combine_kat():
    top1 = {
        "source": "reference tests/test_combine.py:20-42",
        "expert_outputs": [[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]],
        "packed_tokenId": [1, 0, 2],
        "packed_topk_weights": [1.0, 1.0, 1.0],
        "num_tokens": 3,
        # out[tokenId[p]] = y[p]
        "expected": [[0.3, 0.4], [0.1, 0.2], [0.5, 0.6]],
    }
    top2 = {
        "source": "reference tests/test_combine.py:54-90",
        "expert_outputs": [[0.1, 0.2], [0.3, 0.4], [0.5, 0.6], [0.1, 0.2], [0.3, 0.4], [0.5, 0.6]],
        "packed_tokenId": [1, 2, 0, 2, 0, 1],
        "packed_topk_weights": [0.3, 0.4, 0.4, 0.5, 0.3, 0.6],
        "num_tokens": 3,
        # token 0: 0.4*[.5,.6] + 0.3*[.3,.4] = [0.29, 0.36]
        # token 1: 0.3*[.1,.2] + 0.6*[.5,.6] = [0.33, 0.42]
        # token 2: 0.4*[.3,.4] + 0.5*[.1,.2] = [0.17, 0.26]
        "expected": [[0.29, 0.36], [0.33, 0.42], [0.17, 0.26]],
    }
    return {"top1": top1, "top2": top2}


if __name__ == "__main__":
    (HERE / "pack_kat.json").write_text(json.dumps(pack_kat(), indent=1) + "\n")
    (HERE / "combine_kat.json").write_text(json.dumps(combine_kat(), indent=1) + "\n")
    print("wrote pack_kat.json, combine_kat.json")
