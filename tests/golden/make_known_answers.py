"""Write ``known_answers.json``: the hand-computable vectors of the reference's tests.

The values are transcribed from the reference's own test files (cited per
entry).  They pin the raw, un-normalised strict-tril semantics: no softmax, no
1/sqrt(d) scale, diagonal excluded, V broadcast over heads.  Expected values
that the reference test states as a formula (``test_bench_gpu_attn.py``) are
evaluated here with exact rational arithmetic.

Run from the repo root:  ``python tests/golden/make_known_answers.py``
"""

from __future__ import annotations

import json
from fractions import Fraction
from pathlib import Path

HERE = Path(__file__).resolve().parent


def _exact_tril(q, k, v):
    """out[i] = sum_{j<i} <q_i, k_j> v_j over nested lists (one slab), exactly."""
    T = len(q)
    Dv = len(v[0])
    out = []
    for i in range(T):
        row = [Fraction(0)] * Dv
        for j in range(i):
            s = sum(Fraction(a) * Fraction(b) for a, b in zip(q[i], k[j]))
            for d in range(Dv):
                row[d] += s * Fraction(v[j][d])
        out.append([float(x) for x in row])
    return out


def _exact_decode(q, k, v):
    """out[t] = sum_s <q_t, k_s> v_s (all past keys valid), exactly."""
    out = []
    for qt in q:
        row = [Fraction(0)] * len(v[0])
        for ks, vs in zip(k, v):
            s = sum(Fraction(a) * Fraction(b) for a, b in zip(qt, ks))
            for d in range(len(vs)):
                row[d] += s * Fraction(vs[d])
        out.append([float(x) for x in row])
    return out


def build() -> dict:
    cases = {}

    # test_attn_bwd_v4_contract.py:13-36 — distinct Q, K; out.sum().backward().
    cases["raw_tril_fwd_bwd"] = {
        "source": "tests/test_attn_bwd_v4_contract.py:13-36",
        "q": [[[[2.0, 0.0], [1.0, 3.0], [4.0, 5.0]]]],
        "k": [[[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]]],
        "v": [[[[2.0], [3.0], [100.0]]]],
        "dout": [[[[1.0], [1.0], [1.0]]]],
        "out": [[[[0.0], [14.0], [124.0]]]],
        "dq": [[[[0.0, 0.0], [2.0, 4.0], [11.0, 16.0]]]],
        "dk": [[[[10.0, 16.0], [12.0, 15.0], [0.0, 0.0]]]],
        "dv": [[[[21.0], [32.0], [0.0]]]],
    }

    # test_attn_bwd_v4_contract.py:238-253 — self attention (Q passed twice),
    # upstream gradient only on the last row; merged dQ + dK.
    cases["self_attn_single_query"] = {
        "source": "tests/test_attn_bwd_v4_contract.py:238-253",
        "q": [[[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]]],
        "v": [[[[2.0], [3.0], [100.0]]]],
        "dout": [[[[0.0], [0.0], [1.0]]]],
        "out": [[[[0.0], [22.0], [151.0]]]],
        "dq_merged": [[[[10.0, 12.0], [15.0, 18.0], [11.0, 16.0]]]],
        "dv": [[[[17.0], [39.0], [0.0]]]],
    }

    # test_decode_contract_v12.py:17-28 — raw decode score x V.
    cases["decode_raw"] = {
        "source": "tests/test_decode_contract_v12.py:17-28",
        "q": [[[[1.0, 1.0]]]],
        "k_past": [[[[1.0, 1.0], [2.0, 1.0]]]],
        "v_past": [[[[5.0], [7.0]]]],
        "out": [[[[31.0]]]],
    }

    # test_bench_gpu_attn.py:788-803 — cold reference inputs; expected is the
    # formula (q @ k^T).tril(-1) @ v, evaluated exactly here.
    q = [[1.0, 2.0], [3.0, -1.0], [2.0, 1.0]]
    k = [[2.0, 1.0], [-1.0, 3.0], [1.0, -2.0]]
    v = [[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]
    cases["bench_cold"] = {
        "source": "tests/test_bench_gpu_attn.py:788-803",
        "q": [[q]],
        "k": [[k]],
        "v": [[v]],
        "out": [[_exact_tril(q, k, v)]],
    }

    # test_bench_gpu_attn.py:806-830 — decode with two heads, broadcast V.
    qd = [[[2.0, 1.0]], [[-1.0, 3.0]]]
    kd = [
        [[1.0, 0.0], [0.0, 3.0], [-1.0, 2.0]],
        [[2.0, 1.0], [1.0, -1.0], [0.0, 2.0]],
    ]
    vd = [[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]
    cases["bench_decode"] = {
        "source": "tests/test_bench_gpu_attn.py:806-830",
        "q": [qd],
        "k_past": [kd],
        "v_past": [[vd]],
        "out": [[_exact_decode(qd[h], kd[h], vd) for h in range(2)]],
    }
    return cases


def main() -> None:
    path = HERE / "known_answers.json"
    path.write_text(json.dumps(build(), indent=1, sort_keys=True) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
