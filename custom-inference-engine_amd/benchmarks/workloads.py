"""Seeded synthetic inputs of the five attention workloads.

All draws come from ``torch.Generator('cpu').manual_seed(seed)`` in fp32 on
the host, in a fixed order, are multiplied by the stated factor, cast to the
workload dtype and only then moved to the device, so every run (and the CPU
oracle) sees bit-identical inputs. Every workload is causal with the default
scale 1/sqrt(D), 32 query heads over 8 kv heads.

  prefill_s128     B=1  S=128    D=64   fp32 N(0,1)            seed 0  (CPU oracle case)
  prefill_s2048    B=4  S=2048   D=64   fp16 N(0,1)/8          seed 1
  decode_b32       B=32 Lq=1 ctx~U{256..4096}  bs=16 fp16 N(0,1)   seed 2
  verify_b8        B=8  Lq=5 ctx~U{1024..8192} bs=16 bf16 N(0,1)   seed 3
  prefill_s16384   B=1  S=16384  D=128  bf16 N(0,1)/sqrt(128)  seed 4
  decode_b32_d128, verify_b8_d128: the two paged workloads at D=128

Paged draw order: context lengths, block permutation, q, K pool, V pool.
Physical block ids are a random permutation of the pool, dealt to the
sequences in order (sequence 0 takes the first ceil(ctx_0/16) ids, ...).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

HQ, HK = 32, 8


@dataclass
class PrefillCase:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    causal: bool = True

    @property
    def flops(self) -> float:
        """Algorithmic FLOPs of causal attention: 4 * B * Hq * D * sum of
        visible keys = 4 B Hq D S(S+1)/2 (QK^T and PV, 2 FLOP per MAC)."""
        B, H, S, D = self.q.shape
        Lk = self.k.shape[2]
        vis = sum(max(0, min(Lk, Lk - S + i + 1)) for i in range(S)) if self.causal else S * Lk
        return 4.0 * B * H * D * vis


@dataclass
class PagedCase:
    name: str
    q: torch.Tensor
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # int32 (B, max_blocks)
    context_lens: torch.Tensor  # int32 (B,)
    causal: bool = True

    @property
    def bytes(self) -> float:
        """Algorithmic HBM bytes: every K and V row of every sequence once,
        q read + o written, the used block-table entries and the lengths."""
        lens = self.context_lens.cpu().long()
        B, Hq, Lq, D = self.q.shape
        bs, Hk = self.k_pool.shape[1], self.k_pool.shape[2]
        elt = self.q.element_size()
        kv = int(lens.sum()) * Hk * D * elt * 2
        qo = 2 * B * Lq * Hq * D * elt
        tbl = int(((lens + bs - 1) // bs).sum()) * 4 + 4 * B
        return float(kv + qo + tbl)

    @property
    def flops(self) -> float:
        lens = self.context_lens.cpu().long()
        B, Hq, Lq, D = self.q.shape
        vis = 0
        for L in lens.tolist():
            vis += sum(max(0, min(L, L - Lq + i + 1)) for i in range(Lq)) if self.causal else Lq * L
        return 4.0 * Hq * D * vis


def _randn(g, shape, factor, dtype):
    return (torch.randn(shape, generator=g, dtype=torch.float32) * factor).to(dtype)


def prefill_case(name: str, B: int, S: int, D: int, dtype: torch.dtype, factor: float, seed: int,
                 device="cpu") -> PrefillCase:
    g = torch.Generator("cpu").manual_seed(seed)
    q = _randn(g, (B, HQ, S, D), factor, dtype)
    k = _randn(g, (B, HK, S, D), factor, dtype)
    v = _randn(g, (B, HK, S, D), factor, dtype)
    return PrefillCase(name, q.to(device), k.to(device), v.to(device))


def paged_case(name: str, B: int, Lq: int, lo: int, hi: int, D: int, dtype: torch.dtype, seed: int,
               block_size: int = 16, device="cpu") -> PagedCase:
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int64)
    nblk = ((lens + block_size - 1) // block_size)
    num_blocks = int(nblk.sum())
    perm = torch.randperm(num_blocks, generator=g)
    q = _randn(g, (B, HQ, Lq, D), 1.0, dtype)
    kp = _randn(g, (num_blocks, block_size, HK, D), 1.0, dtype)
    vp = _randn(g, (num_blocks, block_size, HK, D), 1.0, dtype)
    width = int(nblk.max())
    bt = torch.zeros((B, width), dtype=torch.int32)
    pos = 0
    for b in range(B):
        n = int(nblk[b])
        bt[b, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    return PagedCase(name, q.to(device), kp.to(device), vp.to(device), bt.to(device),
                     lens.to(torch.int32).to(device))


def prefill_s128(device="cpu", dtype=torch.float32) -> PrefillCase:
    return prefill_case("prefill_s128", 1, 128, 64, dtype, 1.0, 0, device)


def prefill_s2048(device="cpu") -> PrefillCase:
    return prefill_case("prefill_s2048", 4, 2048, 64, torch.float16, 1.0 / 8.0, 1, device)


def decode_b32(device="cpu") -> PagedCase:
    return paged_case("decode_b32", 32, 1, 256, 4096, 64, torch.float16, 2, device=device)


def verify_b8(device="cpu") -> PagedCase:
    return paged_case("verify_b8", 8, 5, 1024, 8192, 64, torch.bfloat16, 3, device=device)


def decode_b32_d128(device="cpu") -> PagedCase:
    """decode_b32 with head_dim 128, the head size of most current models."""
    return paged_case("decode_b32_d128", 32, 1, 256, 4096, 128, torch.float16, 2, device=device)


def verify_b8_d128(device="cpu") -> PagedCase:
    """verify_b8 with head_dim 128."""
    return paged_case("verify_b8_d128", 8, 5, 1024, 8192, 128, torch.bfloat16, 3, device=device)


def prefill_s16384(device="cpu") -> PrefillCase:
    return prefill_case("prefill_s16384", 1, 16384, 128, torch.bfloat16, 1.0 / math.sqrt(128), 4, device)


WORKLOADS = {
    "prefill_s128": prefill_s128,
    "prefill_s2048": prefill_s2048,
    "decode_b32": decode_b32,
    "verify_b8": verify_b8,
    "prefill_s16384": prefill_s16384,
    "decode_b32_d128": decode_b32_d128,
    "verify_b8_d128": verify_b8_d128,
}
