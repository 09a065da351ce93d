"""Pins the oracle's restatement of the reference's rotary embedding
(oracle/rope_ref.py <- kernels/ref/rope_apply_ref.py:6-53) and checks, on the
CPU, the package's own table builder and the argument validation of the RoPE
entry points of the C ABI.

Pinning: the reference's own known answers (tests/kernels/test_rope_ref.py,
tests/model/test_rope.py), a float64 closed form of the rotation as a
complex multiplication (x1 + i x2) * e^(i p theta^(-2j/D)) with pairs
(j, j + D/2), additivity of angles, and the single rounding at the end.
Planted mistakes (interleaved pairs, the opposite rotation, a wrong
frequency, ignored positions, products in half precision) must each fail one
of these checks."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import build_rope_cache_ref, rope_ref

# ---- the reference's known answers ---------------------------------------


def test_identity_at_position_zero():
    # tests/kernels/test_rope_ref.py:9-14, tests/model/test_rope.py:9-13
    cos, sin = build_rope_cache_ref(8, 16)
    x = torch.randn(1, 2, 1, 16)
    assert torch.allclose(rope_ref(x, cos, sin, positions=torch.tensor([0])), x, atol=1e-6)


def test_shape_and_pairwise_norm_preserved():
    # tests/kernels/test_rope_ref.py:17-29
    torch.manual_seed(0)
    cos, sin = build_rope_cache_ref(32, 16)
    x = torch.randn(2, 4, 5, 16)
    y = rope_ref(x, cos, sin)
    assert y.shape == x.shape
    assert torch.allclose(x[..., :8] ** 2 + x[..., 8:] ** 2, y[..., :8] ** 2 + y[..., 8:] ** 2, atol=1e-5)


def test_different_positions_differ():
    # tests/model/test_rope.py:16-22
    cos, sin = build_rope_cache_ref(32, 16)
    x = torch.randn(1, 2, 1, 16)
    assert not torch.allclose(rope_ref(x, cos, sin, torch.tensor([0])), rope_ref(x, cos, sin, torch.tensor([5])))


# ---- closed forms ----------------------------------------------------------


def _closed_form(x: np.ndarray, pos: np.ndarray, theta: float, c=None, s=None) -> np.ndarray:
    """float64 rotation of x (..., L, D) at pos (L,): pair j = (x[j], x[j+D/2])
    as the complex number x[j] + i x[j+D/2], times e^(i pos theta^(-2j/D)) (or
    times c + i s when table values are given)."""
    D = x.shape[-1]
    h = D // 2
    if c is None:
        ang = pos[:, None].astype(np.float64) * theta ** (-2.0 * np.arange(h) / D)[None, :]
        c, s = np.cos(ang), np.sin(ang)
    z = (x[..., :h] + 1j * x[..., h:]) * (c + 1j * s)
    return np.concatenate([z.real, z.imag], axis=-1)


def rope_failures(build, apply) -> list[str]:
    """Every check the oracle must pass; returns the names of failed ones."""
    bad = []
    g = torch.Generator().manual_seed(5)
    for D, theta in ((16, 10000.0), (64, 10000.0), (128, 500000.0)):
        cos, sin = build(4096, D, theta)
        # 1. the table against the float64 angles (fp32 angle rounding < 1e-3)
        j = np.arange(D // 2)
        ang = np.arange(4096)[:, None] * theta ** (-2.0 * j / D)[None, :]
        if (np.abs(cos.double().numpy() - np.cos(ang)).max() > 1e-3 or
                np.abs(sin.double().numpy() - np.sin(ang)).max() > 1e-3):
            bad.append(f"table D={D}")
        # 2. the rotation of fp32 x against the complex product with the same table values
        x = torch.randn(2, 3, 7, D, generator=g)
        pos = torch.tensor([0, 1, 2, 100, 777, 4000, 4095])
        want = _closed_form(x.double().numpy(), pos.numpy(), theta, cos[pos].double().numpy(),
                            sin[pos].double().numpy())
        if np.abs(apply(x, cos, sin, pos).double().numpy() - want).max() > 1e-5:
            bad.append(f"rotation D={D}")
        # 3. (B, L) positions equal per-batch (L,) calls
        pb = torch.stack([pos, pos.flip(0)])
        y = apply(x, cos, sin, pb)
        if not (torch.equal(y[0:1], apply(x[0:1], cos, sin, pos)) and
                torch.equal(y[1:2], apply(x[1:2], cos, sin, pos.flip(0)))):
            bad.append(f"batched positions D={D}")
        # 4. angles add: rot(rot(x, p1), p2) == rot(x, p1 + p2)
        p1, p2 = torch.tensor([3, 10, 20]), torch.tensor([5, 30, 40])
        x3 = x[:, :, :3]
        if (apply(apply(x3, cos, sin, p1), cos, sin, p2) - apply(x3, cos, sin, p1 + p2)).abs().max() > 1e-4:
            bad.append(f"additivity D={D}")
        # 5. fp16 x: fp32 arithmetic, one rounding at the end
        xh = (x * 4).half()
        if not torch.equal(apply(xh, cos, sin, pos), apply(xh.float(), cos, sin, pos).half()):
            bad.append(f"single rounding D={D}")
        # 6. against the closed form with exact angles (pins the frequencies)
        if np.abs(apply(x, cos, sin, pos).double().numpy() -
                  _closed_form(x.double().numpy(), pos.numpy(), theta)).max() > 1e-2:
            bad.append(f"frequencies D={D}")
    return bad


def test_oracle_passes_every_check():
    assert rope_failures(build_rope_cache_ref, rope_ref) == []


def _interleaved(x, cos, sin, positions=None):
    B, H, L, D = x.shape
    pos = torch.arange(L) if positions is None else positions
    c = cos[pos].reshape(-1 if pos.dim() == 2 else 1, 1, L, D // 2)
    s = sin[pos].reshape(-1 if pos.dim() == 2 else 1, 1, L, D // 2)
    a, b = x[..., 0::2].float(), x[..., 1::2].float()
    out = torch.empty(x.shape, dtype=torch.float32)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out.to(x.dtype)


def _wrong_freq(n, D, theta):
    inv = 1.0 / (theta ** (torch.arange(0, D // 2, dtype=torch.float32) / D))
    ang = torch.outer(torch.arange(n, dtype=torch.float32), inv)
    return ang.cos(), ang.sin()


def _half_math(x, cos, sin, positions=None):
    if x.dtype == torch.float32:
        return rope_ref(x, cos, sin, positions)
    B, H, L, D = x.shape
    pos = torch.arange(L) if positions is None else positions
    c = cos[pos].to(x.dtype).reshape(-1 if pos.dim() == 2 else 1, 1, L, D // 2)
    s = sin[pos].to(x.dtype).reshape(-1 if pos.dim() == 2 else 1, 1, L, D // 2)
    x1, x2 = x[..., :D // 2], x[..., D // 2:]
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1)


MUTANTS = {
    "interleaved pairs": (build_rope_cache_ref, _interleaved),
    "opposite rotation": (build_rope_cache_ref, lambda x, c, s, p=None: rope_ref(x, c, -s, p)),
    "wrong frequency": (_wrong_freq, rope_ref),
    "positions ignored": (build_rope_cache_ref, lambda x, c, s, p=None: rope_ref(x, c, s, None)),
    "half-precision products": (build_rope_cache_ref, _half_math),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistakes_are_caught(name):
    build, apply = MUTANTS[name]
    assert rope_failures(build, apply), f"mutant '{name}' passed every check"


# ---- tables cast to the activation dtype ------------------------------------
#
# The reference engine runs with RotaryEmbedding's cos / sin cast to fp16 or
# bf16 (cast_non_quantized_params, engine/runtime.py:22-37). apply_rotary_ref
# then multiplies and adds 16-bit tensors: each operation's result is rounded
# to the 16-bit type. Independent restatements of that arithmetic: numpy's
# float16 (each operation computed in float32 and rounded to half), and for
# bfloat16 an fp32 computation rounded to bfloat16 by integer bit arithmetic
# (nearest even); the float64 rotation with the same table values must lie
# within the bound the four roundings allow.


def _bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned as float32 (finite inputs)."""
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def _numpy_16bit(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> np.ndarray:
    """apply_rotary_ref's expression with every operation rounded to x's
    16-bit type; c, s already indexed and broadcastable (numpy only)."""
    h = x.shape[-1] // 2
    if x.dtype == torch.float16:
        x1, x2 = x[..., :h].numpy(), x[..., h:].numpy()
        cn, sn = c.numpy(), s.numpy()
        out = np.concatenate([x1 * cn - x2 * sn, x1 * sn + x2 * cn], axis=-1)
        return out.astype(np.float32)
    f = lambda t: t.float().numpy()  # noqa: E731 (bf16 -> fp32 is exact)
    x1, x2, cn, sn = f(x[..., :h]), f(x[..., h:]), f(c), f(s)
    r = _bf16_round
    return np.concatenate([r(r(x1 * cn) - r(x2 * sn)), r(r(x1 * sn) + r(x2 * cn))], axis=-1)


def half_table_failures(apply) -> list[str]:
    bad = []
    g = torch.Generator().manual_seed(9)
    for dt, u, tiny in ((torch.float16, 2.0 ** -11, 2.0 ** -24), (torch.bfloat16, 2.0 ** -8, 0.0)):
        for D in (16, 64, 128):
            cos32, sin32 = build_rope_cache_ref(4096, D)
            cos, sin = cos32.to(dt), sin32.to(dt)
            x = (torch.randn(2, 3, 9, D, generator=g) * 3).to(dt)
            pos = torch.tensor([0, 1, 2, 7, 100, 777, 2048, 4000, 4095])
            got = apply(x, cos, sin, pos)
            c, s = cos[pos].reshape(1, 1, 9, D // 2), sin[pos].reshape(1, 1, 9, D // 2)
            # 1. an independent evaluation of the 16-bit arithmetic
            if not np.array_equal(got.float().numpy(), _numpy_16bit(x, c, s)):
                bad.append(f"16-bit arithmetic {dt} D={D}")
            # 2. the reference's own expression evaluated by torch on 16-bit tensors
            h = D // 2
            lit = torch.cat([x[..., :h] * c - x[..., h:] * s, x[..., :h] * s + x[..., h:] * c], -1).to(dt)
            if not torch.equal(got, lit):
                bad.append(f"torch expression {dt} D={D}")
            # 3. float64 rotation with the same table values, within four roundings
            x1, x2 = x[..., :h].double(), x[..., h:].double()
            cd, sd = c.double(), s.double()
            exact = torch.cat([x1 * cd - x2 * sd, x1 * sd + x2 * cd], -1)
            mag = torch.cat([(x1 * cd).abs() + (x2 * sd).abs(), (x1 * sd).abs() + (x2 * cd).abs()], -1)
            if ((got.double() - exact).abs() > 2.01 * u * mag + 3 * tiny).any():
                bad.append(f"rounding bound {dt} D={D}")
            # 4. (B, L) positions equal per-batch (L,) calls
            pb = torch.stack([pos, pos.flip(0)])
            y = apply(x, cos, sin, pb)
            if not (torch.equal(y[0:1], apply(x[0:1], cos, sin, pos)) and
                    torch.equal(y[1:2], apply(x[1:2], cos, sin, pos.flip(0)))):
                bad.append(f"batched positions {dt} D={D}")
    # 5. a mixed pair (fp16 x, bf16 tables) is promoted to fp32: the same as fp32 tables holding those values
    cos32, sin32 = build_rope_cache_ref(512, 64)
    cb, sb = cos32.bfloat16(), sin32.bfloat16()
    x = torch.randn(1, 2, 5, 64, generator=g).half()
    pos = torch.tensor([0, 3, 9, 300, 511])
    if not torch.equal(apply(x, cb, sb, pos), apply(x, cb.float(), sb.float(), pos)):
        bad.append("mixed fp16 x bf16 tables")
    return bad


def test_oracle_with_cast_tables_passes_every_check():
    assert half_table_failures(rope_ref) == []


def _fp32_math_always(x, cos, sin, positions=None):
    # the arithmetic of fp32 tables whatever the table type (tables widened, one rounding)
    return rope_ref(x, cos.float(), sin.float(), positions)


def _fma_products(x, cos, sin, positions=None):
    # difference / sum taken from unrounded products, rounded once to the 16-bit type
    B, H, L, D = x.shape
    pos = torch.arange(L) if positions is None else positions
    c = cos[pos].float().reshape(-1 if pos.dim() == 2 else 1, 1, L, D // 2)
    s = sin[pos].float().reshape(-1 if pos.dim() == 2 else 1, 1, L, D // 2)
    x1, x2 = x[..., :D // 2].float(), x[..., D // 2:].float()
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1).to(x.dtype)


HALF_MUTANTS = {
    "fp32 arithmetic for 16-bit tables": _fp32_math_always,
    "unrounded products": _fma_products,
    "opposite rotation": lambda x, c, s, p=None: rope_ref(x, c, -s, p),
}


@pytest.mark.parametrize("name", sorted(HALF_MUTANTS))
def test_planted_mistakes_with_cast_tables_are_caught(name):
    assert half_table_failures(HALF_MUTANTS[name]), f"mutant '{name}' passed every check"


def test_module_cast_like_the_reference_engine():
    """RotaryEmbedding after the reference engine's cast (every floating
    buffer to the activation dtype, engine/runtime.py:35-37) keeps its
    16-bit tables, and the oracle then rotates with 16-bit arithmetic."""
    from engine.model.rope import RotaryEmbedding

    emb = RotaryEmbedding(64, 256)
    for name, b in list(emb.named_buffers(recurse=False)):
        if b.is_floating_point():
            setattr(emb, name, b.to(torch.float16))
    assert emb.cos.dtype == torch.float16 and emb.tables[0].dtype == torch.float16
    x = torch.randn(1, 2, 4, 64).half()
    pos = torch.tensor([1, 2, 3, 200])
    c, s = emb.cos[pos].reshape(1, 1, 4, 32), emb.sin[pos].reshape(1, 1, 4, 32)
    assert np.array_equal(rope_ref(x, emb.cos, emb.sin, pos).float().numpy(), _numpy_16bit(x, c, s))


# ---- the package's host side ------------------------------------------------


@pytest.mark.parametrize("n,D,theta", [(64, 16, 10000.0), (8192, 128, 10000.0), (4096, 256, 500000.0)])
def test_package_tables_equal_the_reference_tables_bitwise(n, D, theta):
    from engine.model.rope import RotaryEmbedding, build_rope_cache

    c, s = build_rope_cache(n, D, theta)
    rc, rs = build_rope_cache_ref(n, D, theta)
    assert c.dtype == torch.float32 and torch.equal(c, rc) and torch.equal(s, rs)
    emb = RotaryEmbedding(D, n, theta)
    assert torch.equal(emb.cos, rc) and torch.equal(emb.sin, rs)


def test_rope_apply_requires_gpu_tensors():
    from engine.model.rope import RotaryEmbedding

    emb = RotaryEmbedding(16, 8)
    with pytest.raises(RuntimeError):
        emb.apply(torch.randn(1, 2, 3, 16).half())


# ---- C ABI validation (no compute call) ------------------------------------

FAKE = 1 << 20


def _st(*s):
    return (ctypes.c_int64 * 4)(*s)


def _rope(**over):
    from engine import _lib

    a = dict(x=FAKE, out=FAKE, xs=_st(4096, 512, 64, 1), os_=_st(4096, 512, 64, 1), pos=None, pbs=0,
             cos=FAKE, sin=FAKE, rows=128, tdt=2, status=None, B=2, H=8, L=8, D=64, dtype=0)
    a.update(over)
    return _lib.load().cie_rope_apply(a["x"], a["out"], a["xs"], a["os_"], a["pos"], a["pbs"], a["cos"], a["sin"],
                                      a["rows"], a["tdt"], a["status"], a["B"], a["H"], a["L"], a["D"], a["dtype"],
                                      None)


@pytest.mark.parametrize("over,code", [
    (dict(D=24), -2), (dict(dtype=2), -3), (dict(cos=0), -1), (dict(sin=FAKE + 4), -1), (dict(rows=0), -1),
    (dict(x=0), -1), (dict(out=FAKE + 2), -1), (dict(xs=_st(4096, 512, 60, 1)), -1), (dict(pbs=-1), -1),
    (dict(B=-1), -1), (dict(tdt=3), -3), (dict(tdt=-1), -3),
])
def test_rope_apply_rejects_bad_arguments(over, code):
    from engine import _lib

    assert _rope(**over) == code
    assert _lib.last_error()


def test_rope_apply_empty_is_a_no_op():
    assert _rope(L=0, x=0, out=0) == 0


def test_fused_rope_entries_validate_tables():
    from engine import _lib

    lib = _lib.load()
    st = _st(8192, 1024, 64, 1)
    rc = lib.cie_flash_fwd_rope(FAKE, FAKE, FAKE, FAKE, st, st, st, st, 1, 8, 2, 16, 16, 64, 0.125, 1, 0,
                                0, FAKE, 16, 2, None, None)
    assert rc == _lib.CIE_EINVAL and "rope" in _lib.last_error()
    rc = lib.cie_flash_fwd_rope(FAKE, FAKE, FAKE, FAKE, st, st, st, st, 1, 8, 2, 16, 16, 64, 0.125, 1, 0,
                                FAKE, FAKE, 16, 5, None, None)
    assert rc == _lib.CIE_EDTYPE and "rope table dtype" in _lib.last_error()
    rc = lib.cie_paged_fwd_rope(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30, _st(2048, 64, 64, 1),
                                _st(8192, 512, 64, 1), _st(8192, 512, 64, 1), _st(2048, 64, 64, 1),
                                4, 32, 8, 1, 64, 100, 16, 25, 0, 0.125, 1, 0, FAKE, FAKE, 0, 2, None)
    assert rc == _lib.CIE_EINVAL and "rope" in _lib.last_error()
    s3 = (ctypes.c_int64 * 3)(512, 64, 1)
    rc = lib.cie_kv_append_rope(FAKE, FAKE, FAKE, FAKE, s3, s3, _st(8192, 512, 64, 1), _st(8192, 512, 64, 1),
                                FAKE, FAKE, FAKE, None, 2, 4, 2, 8, 64, 100, 16, 25, 0,
                                FAKE, FAKE, 64, 0, FAKE + 2, s3, None)
    assert rc == _lib.CIE_EINVAL and "k_out" in _lib.last_error()
