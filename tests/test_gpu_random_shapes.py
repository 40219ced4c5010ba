"""Seeded sweep over the supported shape matrix against the fp64 oracle.

Each case draws its cache type, head dim, block size, GQA group, number of
kv heads, batch, lengths (with block-, partition- and chunk-edge values
mixed in) and softmax scale from a fixed seed, within what the library
supports: a (block, head) tile of whole 1 KiB loads (head_dim * block_size
/ x a multiple of 64, x = 16 bytes / element), groups 1, 2 and 4, prefill
over 16-bit caches, fp8 decode at head dims 64 / 128. The softmax scale is
drawn within 0.5-1.5 x 1/sqrt(head_dim) (vASR uses exactly 1/sqrt(head_dim))
and fp8's k_scale, which scales the logits too, within 0.3-1.5: at 2.3-2.8
times the default logit scale the f32 and f16 paths drew elements up to 1.5
times the element-wise bound while their error stayed at 1e-6 (f32) and
1e-3 (f16) of the output's largest magnitude, the types' own rounding
against the fp64 oracle. The same acceptance tolerances as the per-op tests
(tests/_util.assert_attention_close). A wider sweep adds f32 queries over
fp8 caches, prefill over f32 and fp8 caches with the denominator's epsilon,
every prefill head dim and block size, the fp8 decode shapes of each query
type and 3 to 8 query heads per kv head; fp8 caches under f32 or bf16
queries are held to the tolerance per output row there (normwise): with
scales other than 1 the reference rounds each dequantised element to the
query type, the kernels scale in f32."""

import numpy as np
import pytest

from oracle import oracle as orc
from tests._util import assert_attention_close, assert_attention_close_normwise
from tests.test_gpu_decode import decode_case
from tests.test_gpu_fp8 import fp8_decode_case
from tests.test_gpu_prefill import prefill_case

pytestmark = pytest.mark.gpu

EDGES = [1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 511, 512, 513, 2047, 2048, 2049]


def _shape(rng, code):
    x = 4 if code == orc.F32 else 8
    while True:
        d = int(rng.choice([64, 96, 128, 192, 256]))
        bs = int(rng.choice([8, 16, 32]))
        if (d * bs // x) % 64 == 0:
            return d, bs


def _heads(rng):
    g = int(rng.choice([1, 2, 4]))
    kvh = int(rng.choice([1, 2, 4, 8]))
    return g * kvh, kvh


def _lens(rng, n, hi):
    lens = rng.integers(1, hi, size=n)
    k = int(rng.integers(0, n + 1))
    lens[:k] = rng.choice(EDGES, size=k)
    return [int(v) for v in np.minimum(lens, hi)]


@pytest.mark.parametrize("case", range(16))
def test_decode_random_shape(device, case):
    rng = np.random.default_rng(5000 + case)
    code = int(rng.choice([orc.F32, orc.BF16, orc.F16]))
    d, bs = _shape(rng, code)
    h, kvh = _heads(rng)
    lens = _lens(rng, int(rng.integers(1, 9)), 3000)
    scale = float(rng.uniform(0.5, 1.5)) * d ** -0.5
    got, want = decode_case(device, code, h, kvh, d, bs, lens, seed=6000 + case, scale=scale)
    assert_attention_close(got, want, code,
                           f"case {case}: code={code} d={d} bs={bs} h={h} kvh={kvh} lens={lens}")


@pytest.mark.parametrize("case", range(12))
def test_prefill_random_shape(device, case):
    rng = np.random.default_rng(7000 + case)
    code = int(rng.choice([orc.BF16, orc.F16]))
    d, bs = _shape(rng, code)
    h, kvh = _heads(rng)
    n = int(rng.integers(1, 5))
    prior = [int(v) for v in rng.integers(0, 600, size=n)]
    new = _lens(rng, n, 300)
    causal = bool(rng.integers(0, 2))
    scale = float(rng.uniform(0.5, 1.5)) * d ** -0.5
    got, want = prefill_case(device, code, h, kvh, d, bs, prior, new, seed=8000 + case,
                             causal=causal, scale=scale)
    assert_attention_close(got, want, code,
                           f"case {case}: code={code} d={d} bs={bs} h={h} kvh={kvh} "
                           f"prior={prior} new={new} causal={causal}")


@pytest.mark.parametrize("case", range(8))
def test_fp8_decode_random_shape(device, case):
    rng = np.random.default_rng(9000 + case)
    code = int(rng.choice([orc.BF16, orc.F16]))
    d, bs = [(64, 16), (64, 32), (128, 8), (128, 16), (128, 32)][int(rng.integers(0, 5))]
    h, kvh = _heads(rng)
    lens = _lens(rng, int(rng.integers(1, 9)), 3000)
    scales = (float(rng.uniform(0.3, 1.5)), float(rng.uniform(0.2, 3.0)))
    got, want = fp8_decode_case(device, code, h, kvh, d, bs, lens, seed=9500 + case,
                                scales=scales)
    assert_attention_close(got, want, code,
                           f"case {case}: code={code} d={d} bs={bs} h={h} kvh={kvh} "
                           f"lens={lens} scales={scales}")


# Query types f32 / bf16 / f16 over f32 / 16-bit / fp8 caches, query heads
# per kv head 1-8 (3 and 6 included), every prefill head dim and block size,
# and the fp8 decode shapes the library takes for its query type.
_FP8_DECODE_16 = [(64, 16), (64, 32), (128, 8), (128, 16), (128, 32), (256, 8), (96, 32),
                  (192, 16), (256, 16)]
_FP8_DECODE_F32 = [(d, bs) for d in (64, 96, 128, 192, 256) for bs in (16, 32)
                   if (d * bs // 16) % 64 == 0 and (d * bs // 16) // 64 <= 6]


@pytest.mark.parametrize("case", range(64))
def test_wide_random_shape(device, case):
    from tests.test_gpu_prefill_vector import vector_case
    rng = np.random.default_rng(11000 + case)
    op = ["decode", "prefill", "fp8_decode", "fp8_prefill"][case % 4]
    code = int(rng.choice([orc.F32, orc.BF16, orc.F16]))
    g = int(rng.choice([1, 2, 3, 4, 6, 8]))
    kvh = int(rng.choice([1, 2, 4, 8]))
    h = g * kvh
    what = f"case {case}: {op} code={code} h={h} kvh={kvh}"
    if op in ("decode", "fp8_decode"):
        lens = _lens(rng, int(rng.integers(1, 9)), 3000)
        if op == "decode":
            d, bs = _shape(rng, code)
            scale = float(rng.uniform(0.5, 1.5)) * d ** -0.5
            got, want = decode_case(device, code, h, kvh, d, bs, lens, seed=12000 + case,
                                    scale=scale)
        else:
            opts = _FP8_DECODE_F32 if code == orc.F32 else _FP8_DECODE_16
            d, bs = opts[int(rng.integers(0, len(opts)))]
            scales = (float(rng.uniform(0.3, 1.5)), float(rng.uniform(0.2, 3.0)))
            got, want = fp8_decode_case(device, code, h, kvh, d, bs, lens, seed=12000 + case,
                                        scales=scales)
        what += f" d={d} bs={bs} lens={lens}"
    else:
        d = int(rng.choice([64, 96, 128, 192, 256]))
        bs = int(rng.choice([8, 16, 32]))
        n = int(rng.integers(1, 5))
        prior = [int(v) for v in rng.integers(0, 600, size=n)]
        new = _lens(rng, n, 300)
        causal = bool(rng.integers(0, 2))
        eps = float(rng.choice([0.0, 1e-6]))
        scale = float(rng.uniform(0.5, 1.5)) * d ** -0.5
        fp8 = op == "fp8_prefill"
        scales = (float(rng.uniform(0.3, 1.5)), float(rng.uniform(0.2, 3.0))) if fp8 else (1.0, 1.0)
        got, want = vector_case(device, code, h, kvh, d, bs, prior, new, seed=12000 + case,
                                causal=causal, eps=eps, fp8=fp8, scales=scales, scale=scale)
        what += f" d={d} bs={bs} prior={prior} new={new} causal={causal} eps={eps}"
    if op.startswith("fp8") and code in (orc.F32, orc.BF16):
        # fp8 with scales other than 1: the kernels scale the logits and the
        # output in f32 where the reference (and the oracle) rounds each
        # dequantised element to the query type first; with bf16 queries
        # that rounding, and with f32 queries the cancelling f32 sums over
        # thousands of tokens, put outputs near zero at up to ~2.6x the
        # element-wise bound (errors below 1 % of the output's largest
        # magnitude): the rows are held to the tolerance normwise
        assert_attention_close_normwise(got, want, code, what)
    else:
        assert_attention_close(got, want, code, what)
