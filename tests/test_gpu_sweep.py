"""Randomized parity sweep: every kernel path of both walks against the oracle.

Each case draws a graph, a walk count around the 64-walk wavefront and queue
chunk and the record walk's few-walks mode (1 .. 40,000), a walk length around the rand-window and long-walk
boundaries (0 .. 129), generated or caller uniforms, a walk offset, int32 or
int64 output, with or without edge ids, and a workspace that selects one
kernel path: for the uniform walk the query's size, edge records, start
records only (CSR walk), the 256-byte LDS header or the 32-byte minimum;
for node2vec each MLXC_N2V_LAYOUT_* size the layout query gives, or the
workspace query's.  node2vec cases also draw p and q, both acceptance rules,
rows sorted, unsorted or detected, and the symmetric-graph hint on symmetric
graphs.  Every case must equal the oracle bit for bit (nodes and edge ids)
and leave no status bit; 2,000 cases per run, from fixed seeds.

Oracle: RandomWalk.cpp:41-60 and BiasedRandomWalk.cpp:20-28,52-100 as
restated in oracle/walk_oracle.c.
"""
import numpy as np
import pytest
import torch

import oracle
from mlx_cluster_amd import _lib, synth

pytestmark = pytest.mark.gpu

# up to 32,768 node2vec walks (on 256 compute units) run in the record walk's
# tail phase from the start; 33,000 and 40,000 take its queue and main loop
N_CHOICES = [1, 2, 63, 64, 65, 127, 129, 1000, 4097, 20000, 33000, 40000]
L_UNIFORM = [0, 1, 2, 3, 4, 5, 7, 8, 15, 16, 17, 31, 32, 33, 40, 63, 64, 65, 80, 127, 128, 129]
L_N2V = [0, 1, 2, 3, 5, 8, 16, 17, 30, 33, 40]
PQ = [(0.5, 2.0), (4.0, 0.25), (1.0, 3.0), (2.0, 0.5), (1.0, 1.0), (0.25, 4.0)]
N2V_LAYOUTS = {"direct": 0, "lds": 1, "csr": 2, "records": 3, "records_hash": 4,
               "records_full": 5, "query": None}


def _unsorted(rowptr, col, seed):
    """The same graph with every row's entries shuffled."""
    rp, cl = rowptr.cpu().numpy(), col.cpu().numpy().copy()
    g = np.random.default_rng(seed)
    for v in range(rp.size - 1):
        a, b = rp[v], rp[v + 1]
        if b - a > 1:
            cl[a:b] = cl[a:b][g.permutation(b - a)]
    return torch.from_numpy(cl).to(col.device)


@pytest.fixture(scope="module")
def graphs(cuda):
    g = {
        "rmat7": synth.rmat_csr(7, 300, seed=3, device=cuda),
        "rmat12": synth.rmat_csr(12, 30000, seed=4, device=cuda),
        "rmat11s": synth.rmat_csr(11, 40000, seed=5, device=cuda, symmetrize=True),
        "rmat16": synth.rmat_csr(16, 600000, seed=6, device=cuda),
        # symmetric, with 4 hub rows of about 3,000 entries (hub bitmaps)
        "bahub": synth.ba_hub_csr(20000, 3, 4, 3000, seed=7, device=cuda),
    }
    g["rmat11s_unsorted"] = (g["rmat11s"][0], _unsorted(*g["rmat11s"], 9))
    g["rmat12_unsorted"] = (g["rmat12"][0], _unsorted(*g["rmat12"], 10))
    return {k: (r, c, r.cpu().numpy(), c.cpu().numpy()) for k, (r, c) in g.items()}


def _outputs(N, L, int32, edges, device):
    dt = torch.int32 if int32 else torch.int64
    n_out = torch.full((N, L + 1), -7, dtype=dt, device=device)
    e_out = torch.full((N, L), -7, dtype=dt, device=device) if edges else None
    n_p = n_out.data_ptr() if n_out.numel() else None
    e_p = e_out.data_ptr() if edges and e_out.numel() else None
    return n_out, e_out, n_p, e_p, (_lib.MLXC_OUT_INT32 if int32 else _lib.MLXC_OUT_INT64)


def _compare(name, ws, n_out, e_out, ref, ref_e, failures):
    torch.cuda.synchronize()
    bits = int(ws[0].item())
    if bits:
        failures.append(f"{name}: status {bits}")
        return
    got = n_out.cpu().numpy().astype(np.int64)
    if not np.array_equal(got, ref):
        at = tuple(np.argwhere(got != ref)[0])
        failures.append(f"{name}: nodes differ first at {at}: {got[at]} vs {ref[at]}")
    elif e_out is not None:
        got_e = e_out.cpu().numpy().astype(np.int64)
        if not np.array_equal(got_e, ref_e):
            at = tuple(np.argwhere(got_e != ref_e)[0])
            failures.append(f"{name}: edge ids differ first at {at}: {got_e[at]} vs {ref_e[at]}")


def _uniform_case(rng, graphs, device, lib, stream, failures):
    gname = str(rng.choice(["rmat7", "rmat12", "rmat16", "bahub", "rmat11s"]))
    rowptr, col, rp, cl = graphs[gname]
    V, E = rp.size - 1, cl.size
    N, L = int(rng.choice(N_CHOICES)), int(rng.choice(L_UNIFORM))
    N = max(1, min(N, 3_000_000 // max(L, 1)))
    seeded = bool(rng.integers(2))
    first = int(rng.choice([0, 0, 5, 1 << 33])) if seeded else 0
    seed = int(rng.integers(1 << 62))
    int32, edges = bool(rng.integers(2)), bool(rng.integers(2))
    mode = str(rng.choice(["query", "records", "csr", "lds", "minimum"]))
    start_h = rng.integers(0, V, N).astype(np.int64)
    rand_h = (oracle.philox_uniform(N * L, seed, first * L) if seeded
              else rng.random(N * L, dtype=np.float32))
    ref, ref_e, st, _ = oracle.uniform_walk(rp, cl, start_h, rand_h, L, with_edges=True)
    assert st == 0
    ws_bytes = {"query": lib.mlxc_random_walk_workspace_bytes(V, E, N, L),
                "records": 256 + 16 * (E + N), "csr": 256 + 16 * N, "lds": 256,
                "minimum": 32}[mode]
    ws = torch.empty((max(ws_bytes, 32) + 7) // 8, dtype=torch.int64, device=device)
    n_out, e_out, n_p, e_p, ot = _outputs(N, L, int32, edges, device)
    start = torch.from_numpy(start_h).to(device)
    if seeded:
        rc = lib.mlxc_random_walk_seeded(rowptr.data_ptr(), V, col.data_ptr(), E,
                                         start.data_ptr(), N, L, seed, first, n_p, e_p, ot,
                                         ws.data_ptr(), ws_bytes, stream)
    else:
        rand = torch.from_numpy(rand_h).to(device)
        rc = lib.mlxc_random_walk(rowptr.data_ptr(), V, col.data_ptr(), E, start.data_ptr(), N,
                                  rand.data_ptr() if rand.numel() else None, L, n_p, e_p, ot,
                                  ws.data_ptr(), ws_bytes, stream)
    name = (f"uniform {gname} N={N} L={L} seeded={seeded} first={first} int32={int32} "
            f"edges={edges} workspace={mode}:{ws_bytes}")
    if rc != _lib.MLXC_OK:
        failures.append(f"{name}: rc {rc} {_lib.last_error()}")
        return
    _compare(name, ws, n_out, e_out, ref, ref_e, failures)


def _n2v_case(rng, graphs, device, lib, stream, failures):
    gname = str(rng.choice(["rmat7", "rmat12", "rmat11s", "bahub", "rmat11s_unsorted",
                            "rmat12_unsorted", "rmat16"]))
    rowptr, col, rp, cl = graphs[gname]
    V, E = rp.size - 1, cl.size
    N, L = int(rng.choice(N_CHOICES[:-1])), int(rng.choice(L_N2V))
    N = max(1, min(N, 400_000 // max(L, 1)))
    p, q = PQ[int(rng.integers(len(PQ)))]
    rule = int(rng.integers(2))
    unsorted = gname.endswith("_unsorted")
    rows = int(rng.choice([_lib.MLXC_ROWS_UNSORTED, _lib.MLXC_ROWS_DETECT] if unsorted else
                          [_lib.MLXC_ROWS_UNSORTED, _lib.MLXC_ROWS_SORTED, _lib.MLXC_ROWS_DETECT]))
    symmetric_graph = gname in ("rmat11s", "bahub")
    if symmetric_graph and rows != _lib.MLXC_ROWS_UNSORTED and rng.integers(2):
        rows |= _lib.MLXC_ROWS_SYMMETRIC
    first = int(rng.choice([0, 0, 7, 1 << 35]))
    seed = int(rng.integers(1 << 62))
    int32, edges = bool(rng.integers(2)), bool(rng.integers(2))
    layout = str(rng.choice(list(N2V_LAYOUTS)))
    start_h = rng.integers(0, V, N).astype(np.int64)
    ref, ref_e, st, _ = oracle.node2vec_walk(rp, cl, start_h, L, p, q, seed, rule=rule,
                                             rows_sorted=not unsorted, with_edges=True,
                                             first_walk=first)
    assert st == 0
    if N2V_LAYOUTS[layout] is None:
        ws_bytes = lib.mlxc_rejection_sampling_workspace_bytes(V, E, N, L, p, q, rule)
    else:
        ws_bytes = lib.mlxc_rejection_sampling_layout_bytes(V, E, N, L, N2V_LAYOUTS[layout])
        if ws_bytes == 0:
            return  # the layout does not apply to these sizes
    ws = torch.empty((max(ws_bytes, 32) + 7) // 8, dtype=torch.int64, device=device)
    n_out, e_out, n_p, e_p, ot = _outputs(N, L, int32, edges, device)
    start = torch.from_numpy(start_h).to(device)
    rc = lib.mlxc_rejection_sampling(rowptr.data_ptr(), V, col.data_ptr(), E, start.data_ptr(),
                                     N, L, p, q, seed, first, rule, rows, n_p, e_p, ot,
                                     ws.data_ptr(), ws_bytes, stream)
    name = (f"node2vec {gname} N={N} L={L} p={p} q={q} rule={rule} rows={rows} first={first} "
            f"int32={int32} edges={edges} layout={layout}:{ws_bytes}")
    if rc != _lib.MLXC_OK:
        failures.append(f"{name}: rc {rc} {_lib.last_error()}")
        return
    _compare(name, ws, n_out, e_out, ref, ref_e, failures)


@pytest.mark.parametrize("seed", [11, 12, 13, 14])
def test_random_cases_match_the_oracle(seed, graphs, cuda):
    rng = np.random.default_rng(seed)
    lib = _lib.load()
    stream = torch.cuda.current_stream(cuda).cuda_stream
    failures = []
    for i in range(500):
        case = _uniform_case if i % 2 == 0 else _n2v_case
        case(rng, graphs, cuda, lib, stream, failures)
    assert not failures, f"{len(failures)} of 500 cases differ:\n" + "\n".join(failures[:10])
