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
(tests/_util.assert_attention_close)."""

import numpy as np
import pytest

from oracle import oracle as orc
from tests._util import assert_attention_close
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
