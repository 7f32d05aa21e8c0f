"""Writes tests/golden/c1_cora_like.npz: configuration 1 inputs and outputs.

Config 1 (BASELINE): a Cora-sized preferential-attachment graph (2,708
nodes, 5,278 undirected pairs -> 10,556 CSR entries), starts = arange(2000),
walk_length = 5, rand = Philox uniforms (seed 1) of shape [2000, 5] — the
shapes of /root/reference/tests/test_random_walk.py:9-36 and
/root/reference/tests/test_rejection_sampling.py:9-33 (p=1, q=3).

Expected outputs come from the CPU oracle (oracle/), which restates the
reference's eval_cpu loops; the fixture freezes them so that a later change
to either side shows up as a diff.  Run from the repo root:
    python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from mlx_cluster_amd import synth  # noqa: E402

N2V_CASES = [  # (name, p, q, rule, seed)
    ("p1_q3_ref", 1.0, 3.0, oracle.RULE_REF_CHAIN, 1),
    ("p1_q3_exact", 1.0, 3.0, oracle.RULE_NODE2VEC_EXACT, 1),
    ("p05_q2_ref", 0.5, 2.0, oracle.RULE_REF_CHAIN, 3),
    ("p4_q025_ref", 4.0, 0.25, oracle.RULE_REF_CHAIN, 5),
    ("p4_q025_exact", 4.0, 0.25, oracle.RULE_NODE2VEC_EXACT, 5),
]


def main():
    rowptr, col = synth.cora_like(seed=0)
    start = np.arange(2000, dtype=np.int64)
    L = 5
    rand = oracle.philox_uniform(2000 * L, seed=1).reshape(2000, L)
    n_out, e_out, st, counts = oracle.uniform_walk(rowptr, col, start, rand, L, with_edges=True)
    assert st == 0
    out = dict(rowptr=rowptr, col=col, start=start, rand=rand, walk_length=np.int64(L),
               uniform_nodes=n_out, uniform_edges=e_out)
    for name, p, q, rule, seed in N2V_CASES:
        n2, e2, st, _ = oracle.node2vec_walk(rowptr, col, start, L, p, q, seed, rule=rule,
                                             with_edges=True)
        assert st == 0
        out[f"n2v_{name}_nodes"] = n2
        out[f"n2v_{name}_edges"] = e2
        out[f"n2v_{name}_params"] = np.array([p, q, rule, seed], dtype=np.float64)
    path = os.path.join(HERE, "c1_cora_like.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes; max degree", int(np.diff(rowptr).max()))


if __name__ == "__main__":
    main()
