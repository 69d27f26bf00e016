"""Float64 decode attention used as the reference for the fused kernel: one query
token per sequence, grouped-query heads (query head h reads kv head h // group),
scale 1/sqrt(head_dim), softmax over the context. Pinned on the CPU by closed
forms in tests/test_attention_reference.py."""

import numpy as np


def attention_f64(q, k, v):
    """q (q_heads, d); k, v (tokens, kv_heads, d) -> (q_heads, d)."""
    group = q.shape[0] // k.shape[1]
    out = np.empty_like(q)
    for qh in range(q.shape[0]):
        kh = k[:, qh // group]
        s = kh @ q[qh] / np.sqrt(q.shape[1])
        p = np.exp(s - s.max())
        out[qh] = (p / p.sum()) @ v[:, qh // group]
    return out
