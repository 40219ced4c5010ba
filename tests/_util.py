"""Helpers shared by the GPU parity tests: numpy <-> torch for 16-bit words,
seeded paged-cache cases and tolerance checks."""

import numpy as np
import torch

from oracle import oracle as orc

TORCH = {orc.F32: torch.float32, orc.BF16: torch.bfloat16, orc.F16: torch.float16}
CODE = {torch.float32: orc.F32, torch.bfloat16: orc.BF16, torch.float16: orc.F16}
# Acceptance tolerances for attention (relative, normwise per row block).
TOL = {orc.F32: 1e-5, orc.BF16: 2e-2, orc.F16: 2e-2}


def to_dev(a: np.ndarray, code: int, device) -> torch.Tensor:
    if code == orc.F32:
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16))
    return t.view(TORCH[code]).to(device)


def to_host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def u32(a, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32)).to(device)


def i64(a, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int64)).to(device)


def random_words(rng, shape, code):
    return orc.from_f32(rng.standard_normal(shape).astype(np.float32), code)


def make_cache(rng, nb, kvh, d, bs, code, zero=False):
    x = 16 // (4 if code == orc.F32 else 2)
    ks, vs = (nb, kvh, d // x, bs, x), (nb, kvh, d, bs)
    if zero:
        dt = np.float32 if code == orc.F32 else np.uint16
        return np.zeros(ks, dtype=dt), np.zeros(vs, dtype=dt)
    return random_words(rng, ks, code), random_words(rng, vs, code)


def block_tables_for(rng, lens, nb, bs, first=1, pad_cols=0):
    need = [(int(L) + bs - 1) // bs for L in lens]
    cols = max(max(need), 1) + pad_cols
    ids = rng.permutation(np.arange(first, nb))
    assert sum(need) <= len(ids), "pool too small"
    bt = np.zeros((len(lens), cols), dtype=np.uint32)
    off = 0
    for s, n in enumerate(need):
        bt[s, :n] = ids[off:off + n]
        off += n
    return bt


# Floor of the elementwise bound, as a fraction of max|want|. An output near
# zero is a sum of terms that cancel; its error is the rounding of those
# terms, not of the result. Measured over the GPU suite (worst element /
# bound): f32 0.50 and f16 0.375 with a floor of 0.03; bf16 0.72 with 0.1
# (1.94 with 0.03), and fp8 caches read with bf16 queries up to 1.00 with
# 0.1: a 5-token context with v_scale 3.1, whose element a CPU emulation of
# the same arithmetic (probabilities rounded to bf16 for P.V, as the
# reference's CUDA kernel does) reproduces at the same ratio.
FLOOR = {orc.F32: 0.03, orc.F16: 0.03, orc.BF16: 0.1}


def assert_attention_close(got_f32: np.ndarray, want_f64: np.ndarray, code: int, what=""):
    """|got - want| <= tol * (|want| + FLOOR * max|want|) per element: relative
    at the stated tolerance (TOL), with a floor for entries near zero."""
    tol = TOL[code]
    want = want_f64.astype(np.float64)
    got = got_f32.astype(np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    scale = np.abs(want).max() if want.size else 0.0
    err = np.abs(got - want)
    bound = tol * (np.abs(want) + FLOOR[code] * scale) + 1e-30
    worst = np.max(err / bound) if err.size else 0.0
    assert worst <= 1.0, (f"{what}: max err {err.max():.3e} exceeds tol {tol} "
                          f"(ratio {worst:.2f}, max|ref| {scale:.3e})")


def attention_errors(got_f32: np.ndarray, want_f64: np.ndarray, code: int):
    """(worst element / element-wise bound of assert_attention_close, worst
    per-row normwise relative error); a row is one output vector along the
    last axis (head_dim)."""
    tol = TOL[code]
    want = want_f64.astype(np.float64)
    got = got_f32.astype(np.float64)
    scale = np.abs(want).max() if want.size else 0.0
    err = np.abs(got - want)
    bound = tol * (np.abs(want) + FLOOR[code] * scale) + 1e-30
    worst = float(np.max(err / bound)) if err.size else 0.0
    num = np.sqrt(((got - want) ** 2).sum(axis=-1))
    den = np.sqrt((want ** 2).sum(axis=-1)) + 1e-300
    return worst, float(np.max(num / den)) if num.size else 0.0


def assert_attention_close_normwise(got_f32: np.ndarray, want_f64: np.ndarray, code: int,
                                    what=""):
    """||got - want||_2 <= tol * ||want||_2 for every output row (one
    (sequence, head) vector of head_dim values), at the stated tolerance
    (TOL): the acceptance bar read normwise, for the regions where single
    elements near zero sit at the rounding of their cancelling terms."""
    tol = TOL[code]
    want = want_f64.astype(np.float64)
    got = got_f32.astype(np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    num = np.sqrt(((got - want) ** 2).sum(axis=-1))
    den = np.sqrt((want ** 2).sum(axis=-1))
    worst = float(np.max(num / np.maximum(den, 1e-300))) if num.size else 0.0
    assert worst <= tol, f"{what}: normwise rel err {worst:.3e} exceeds tol {tol}"
