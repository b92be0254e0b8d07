"""Exact k-NN and recall gates shared by the GPU search tests.

exact_knn is independent of the GPU path and of the oracle's search: fp32
GEMM candidates (k + 64 per query, numpy), re-scored in fp64 and ordered by
(distance, id).

assert_recall_not_below is the graph-search parity gate: the GPU's recall@k
must be at least the reference search's on the same graph, navigation nodes
and itopk.  The comparison is paired over queries: with h_i the GPU's minus
the reference's hits on query i, the mean of h over Q queries must not lie
more than z = 3 standard errors (sd(h) / sqrt(Q)) below zero.  A GPU that is
worse by a margin wider than that noise fails; an exact tie passes.
"""
import numpy as np


def exact_knn(base: np.ndarray, qs: np.ndarray, k: int, extra: int = 64) -> np.ndarray:
    n = base.shape[0]
    norms = np.einsum("ij,ij->i", base, base)
    keep = min(k + extra, n)
    out = np.empty((qs.shape[0], k), np.int64)
    for q0 in range(0, qs.shape[0], 1000):
        qb = qs[q0:q0 + 1000]
        approx = norms[None, :] - 2.0 * (qb @ base.T)
        cand = np.argpartition(approx, keep - 1, axis=1)[:, :keep]
        for r in range(qb.shape[0]):
            c = cand[r]
            d = ((base[c].astype(np.float64) - qb[r].astype(np.float64)) ** 2).sum(1)
            out[q0 + r] = c[np.lexsort((c, d))[:k]]
    return out


def hits(nbr: np.ndarray, gt: np.ndarray, k: int, whole_rows: bool = False) -> np.ndarray:
    """Per row, how many of gt's first k ids are among nbr's first k (or,
    with whole_rows, anywhere in nbr's row: a graph row's neighbour recall)."""
    return np.array([len(set((nbr[i] if whole_rows else nbr[i, :k]).tolist()) & set(gt[i, :k].tolist()))
                     for i in range(len(nbr))], np.float64)


def recall(nbr: np.ndarray, gt: np.ndarray, k: int) -> float:
    return float(hits(nbr, gt, k).mean() / k)


def assert_recall_not_below(nbr: np.ndarray, ref_nbr: np.ndarray, gt: np.ndarray, k: int, label: str = "",
                            z: float = 3.0, whole_rows: bool = False) -> None:
    h_gpu, h_ref = hits(nbr, gt, k, whole_rows), hits(ref_nbr, gt, k, whole_rows)
    diff = h_gpu - h_ref
    se = diff.std(ddof=1) / np.sqrt(len(diff)) if len(diff) > 1 else 0.0
    r_gpu, r_ref = h_gpu.mean() / k, h_ref.mean() / k
    print(f"{label}: recall@{k} gpu {r_gpu:.4f} reference {r_ref:.4f} "
          f"(paired difference {diff.mean() / k:+.4f}, standard error {se / k:.4f}, {len(diff)} queries)")
    assert diff.mean() >= -z * se, (label, r_gpu, r_ref, se / k)
