"""Oracle: scaled dot-product attention (frame / global attention of VGGT).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Not in the reference (the VGGT model graph lives in the external vggt-hf;
the reference extension's attention op is an LLM decode kernel that is out
of scope).  Restated as torch's SDPA without mask: for each sequence,
head and query, out = softmax(q k^T * scale) v, evaluated here in float64.
``rows`` restricts the computation to a subset of query rows so that full
sizes (43,968-token global attention) stay cheap: each selected row still
attends to every key of its sequence.

Pinning (tests/test_oracle_attention.py): uniform scores give the mean of
v; a dominant key returns that key's value; softmax rows sum to one;
agreement with a direct exp/normalise loop on a tiny case.
"""
from __future__ import annotations

import numpy as np


def attention_ref(q, k, v, B: int, L: int, scale: float = 0.125, rows=None, q_rows: bool = False) -> np.ndarray:
    """q, k, v: (B*L, H, D) arrays (``q_rows``: q holds only the selected rows,
    (len(rows), H, D)).  Returns float64 (len(rows) or B*L, H, D); the
    products run per head as float64 matrix products."""
    k = np.asarray(k)
    v = np.asarray(v)
    T, H, D = k.shape
    rows = np.arange(T) if rows is None else np.asarray(rows)
    q = np.asarray(q)
    out = np.empty((len(rows), H, D))
    for seq in range(B):
        sel = np.nonzero((rows >= seq * L) & (rows < (seq + 1) * L))[0]
        if len(sel) == 0:
            continue
        ks = np.asarray(k[seq * L:(seq + 1) * L], np.float64).transpose(1, 2, 0)   # (H, D, L)
        vs = np.asarray(v[seq * L:(seq + 1) * L], np.float64).transpose(1, 0, 2)   # (H, L, D)
        qs = np.asarray(q[sel] if q_rows else q[rows[sel]], np.float64).transpose(1, 0, 2)  # (H, n, D)
        s = np.matmul(qs, ks) * scale                                            # (H, n, L)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[sel] = np.matmul(p, vs).transpose(1, 0, 2)
    return out
