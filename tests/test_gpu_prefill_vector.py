"""GPU parity of the chunked prefill on the vector-ALU kernel against the fp64
oracle: the configurations the MFMA kernel is not built for.

* f32 queries over f32 caches and over fp8 caches with scales, the Metal
  prefill's `float` and `float, uint8_t` instances
  (prefill_paged_attn.metal:1606, 1610; F32 dispatch at
  vasr-paged-attn/src/metal/kernels/mod.rs:119-137): rel 1e-5, causal
  (flash varlen, eps 0) and not (the Metal kernel's 1e-6 and a large eps),
  every head dim and block size, ragged lengths, absent blocks;
* numbers of query heads per kv head the MFMA kernel does not take (3, 8,
  16; the Metal dispatch takes any, mod.rs:145-283), 16-bit and fp8;
* 16-bit and fp8 head-dim / block-size pairs without whole 1 KiB DMAs."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (assert_attention_close, block_tables_for, make_cache, random_words,
                         to_dev, to_host, u32)

pytestmark = pytest.mark.gpu


def f8_dev(a, device):
    return torch.from_numpy(a).to(device).view(torch.float8_e4m3fn)


def vector_case(device, code, h, kvh, d, bs, prior, qlens, seed, causal=True, eps=None, fp8=False,
                scales=(1.0, 1.0), mutate_bt=None, scale=None):
    rng = np.random.default_rng(seed)
    prior = np.asarray(prior, dtype=np.int64)
    qlens = np.asarray(qlens, dtype=np.int64)
    lens = prior + qlens
    nb = int(sum((int(L) + bs - 1) // bs for L in lens)) + 8
    if fp8:
        kc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d // 16, bs, 16)) * 2)
                              .astype(np.float32))
        vc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d, bs)) * 2).astype(np.float32))
        kc_d, vc_d = f8_dev(kc, device), f8_dev(vc, device)
        ks = torch.tensor([scales[0]], dtype=torch.float32, device=device)
        vs = torch.tensor([scales[1]], dtype=torch.float32, device=device)
    else:
        kc, vc = make_cache(rng, nb, kvh, d, bs, code)
        kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
        ks = vs = None
    bt = block_tables_for(rng, [max(int(L), 1) for L in lens], nb, bs)
    if mutate_bt is not None:
        mutate_bt(bt)
    q = random_words(rng, (int(qlens.sum()), h, d), code)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    lens32 = lens.astype(np.uint32)
    scale = d ** -0.5 if scale is None else scale
    eps = (0.0 if causal else 1e-6) if eps is None else eps
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), kc_d, vc_d, u32(bt, device), u32(lens32, device),
        u32(cu, device), ks, vs, scale, 1.0, causal=causal, denom_eps=eps)
    torch.cuda.synchronize()
    want = orc.prefill_attention(q, kc, vc, bt, lens32, cu, scale, causal=causal, dtype=code,
                                 eps=eps, kv_dtype=orc.FP8 if fp8 else None,
                                 k_scale=scales[0], v_scale=scales[1])
    return orc.to_f32(to_host(out), code), want


PRIOR = [0, 5, 31, 100, 0, 333, 16]
NEW = [1, 31, 32, 33, 129, 70, 3]


@pytest.mark.parametrize("d", [64, 96, 128, 192, 256])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("causal,eps", [(True, 0.0), (False, 1e-6), (True, 1e-6), (False, 0.0)])
def test_prefill_f32(device, d, bs, causal, eps):
    got, want = vector_case(device, orc.F32, 16, 8, d, bs, PRIOR, NEW,
                            seed=d + bs + 2 * causal + int(eps > 0), causal=causal, eps=eps)
    assert_attention_close(got, want, orc.F32, f"f32 d={d} bs={bs} causal={causal} eps={eps}")


@pytest.mark.parametrize("d,bs", [(128, 16), (128, 8), (64, 32), (256, 16), (96, 32)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.37, 2.5)])
def test_prefill_f32_query_fp8_cache(device, d, bs, causal, scales):
    got, want = vector_case(device, orc.F32, 16, 8, d, bs, PRIOR, NEW, seed=d + bs + causal,
                            causal=causal, fp8=True, scales=scales)
    assert_attention_close(got, want, orc.F32, f"f32/fp8 d={d} bs={bs} causal={causal}")


@pytest.mark.parametrize("h,kvh", [(24, 8), (64, 8), (16, 1), (32, 2), (8, 8)])
@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
def test_prefill_query_heads_per_kv_head(device, h, kvh, code):
    """3, 8 and 16 query heads per kv head (and 1 for f32) on the vector
    kernel; 16-bit with 1 / 2 / 4 stays on the MFMA kernel."""
    got, want = vector_case(device, code, h, kvh, 128, 16, [7, 0, 260], [40, 65, 17],
                            seed=h + kvh + code)
    assert_attention_close(got, want, code, f"h={h} kvh={kvh} code={code}")


@pytest.mark.parametrize("code,d,bs,fp8", [(orc.BF16, 96, 8, False), (orc.F16, 96, 8, False),
                                           (orc.BF16, 96, 16, True), (orc.F16, 64, 8, True),
                                           (orc.BF16, 192, 8, True)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_vector_16bit_shapes(device, code, d, bs, fp8, causal):
    """Head-dim / block-size pairs whose (block, head) tile is not a whole
    number of 1 KiB DMAs (no MFMA instance) on the vector kernel."""
    got, want = vector_case(device, code, 16, 8, d, bs, PRIOR, NEW, seed=d + bs + fp8 + causal,
                            causal=causal, fp8=fp8, scales=(0.8, 1.3) if fp8 else (1.0, 1.0))
    assert_attention_close(got, want, code, f"code={code} d={d} bs={bs} fp8={fp8}")


def test_prefill_f32_absent_blocks_and_large_scales(device):
    """Table entries outside the pool are skipped (their keys do not count);
    logit scales of 3 and 10 times 1/sqrt(d) (normwise at 10x, where single
    elements near zero sit at the f32 rounding of logits of size ~40)."""
    def corrupt(bt):
        bt[1, 0] = 1 << 30
        bt[3, 2] = 0xffffffff

    got, want = vector_case(device, orc.F32, 16, 8, 128, 16, PRIOR, NEW, seed=5,
                            mutate_bt=corrupt)
    assert_attention_close(got, want, orc.F32, "absent blocks")
    for factor in (3.0, 10.0):
        got, want = vector_case(device, orc.F32, 16, 8, 128, 16, PRIOR, NEW, seed=6,
                                scale=factor * 128 ** -0.5)
        num = np.sqrt(((got - want) ** 2).sum(axis=-1))
        den = np.sqrt((want ** 2).sum(axis=-1))
        assert np.max(num / np.maximum(den, 1e-300)) <= 1e-5, f"scale x{factor}"


def test_prefill_f32_row_without_keys_and_empty_sequences(device):
    """Non-causal rows of a sequence whose every block is absent see no key:
    zeros; sequences without new tokens write nothing."""
    def absent(bt):
        bt[2, :] = 1 << 30

    got, want = vector_case(device, orc.F32, 16, 8, 64, 8, [10, 0, 40, 3], [5, 0, 7, 9], seed=8,
                            causal=False, mutate_bt=absent)
    assert_attention_close(got, want, orc.F32, "no keys")
    assert not np.any(got[5:12])
