"""fp64 numpy brute-force attention, written independently of the torch
restatement (no matmul, no softmax routine: explicit per-row scores, a
max-subtracted exponential and a weighted sum).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). Sized for tiny inputs.

Semantics follow ``kernels/ref/flash_attention_ref.py:8-56``: query head ``h``
uses kv head ``h // (H // Hk)``; under ``causal`` row ``i`` sees keys
``j <= Lk - Lq + i``; default scale ``1/sqrt(D)``; a row with keys but none
visible is NaN (softmax of an all ``-inf`` row); ``Lk == 0`` yields zeros
(an empty softmax times an empty V).
"""

from __future__ import annotations

import math

import numpy as np


def attention_brute_f64(q, k, v, causal: bool = False, scale: float | None = None) -> np.ndarray:
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, Lq, D = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    assert H % Hk == 0
    group = H // Hk
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, H, Lq, D), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            kh = h // group
            for i in range(Lq):
                if Lk == 0:
                    continue
                last = Lk - 1 if not causal else Lk - Lq + i
                if last < 0:
                    out[b, h, i, :] = np.nan
                    continue
                s = np.empty(last + 1)
                for j in range(last + 1):
                    acc = 0.0
                    for d in range(D):
                        acc += q[b, h, i, d] * k[b, kh, j, d]
                    s[j] = acc * scale
                m = s.max()
                w = np.exp(s - m)
                out[b, h, i, :] = (w[:, None] * v[b, kh, :last + 1, :]).sum(axis=0) / w.sum()
    return out


def paged_attention_brute_f64(q, k_pool, v_pool, block_tables, context_lens, causal=True, scale=None):
    """Paged form: token ``t`` of sequence ``b`` is row
    ``pool[block_tables[b][t // bs], t % bs]``."""
    q = np.asarray(q, dtype=np.float64)
    kp = np.asarray(k_pool, dtype=np.float64)
    vp = np.asarray(v_pool, dtype=np.float64)
    bt = np.asarray(block_tables)
    lens = np.asarray(context_lens)
    B = q.shape[0]
    bs = kp.shape[1]
    outs = []
    for b in range(B):
        L = int(lens[b])
        kd = np.stack([kp[bt[b][t // bs], t % bs] for t in range(L)]) if L else np.zeros((0,) + kp.shape[2:])
        vd = np.stack([vp[bt[b][t // bs], t % bs] for t in range(L)]) if L else np.zeros((0,) + vp.shape[2:])
        outs.append(attention_brute_f64(q[b:b + 1], kd.transpose(1, 0, 2)[None], vd.transpose(1, 0, 2)[None],
                                        causal=causal, scale=scale)[0])
    return np.stack(outs)
