"""The committed golden fixtures (tests/golden/*.npz) against the CPU oracle.

Every fixture holds the seeded inputs of one small case and the outputs the
oracle gave for them when the fixture was written
(tests/golden/make_golden.py). Here the inputs are regenerated from the
seed and must equal the stored ones bit for bit, and the oracle's outputs
over the stored inputs must equal the stored outputs: exactly for cache
bytes, gathered rows and token ids, to 1e-12 of the largest magnitude for
the float64 attention outputs. A change of the oracle, or of its build,
that moves any result shows here against the committed vectors."""

import json
import os

import numpy as np
import pytest

from tests.golden import make_golden as mg


@pytest.mark.parametrize("name", sorted(mg.CASES))
def test_fixture_reproduced_by_oracle(name):
    p, inputs, want = mg.load(name)
    assert p == json.loads(json.dumps(mg.CASES[name], sort_keys=True))
    fresh = mg.make_inputs(p)
    assert sorted(fresh) == sorted(inputs)
    for k, v in fresh.items():
        assert v.dtype == inputs[k].dtype and v.shape == inputs[k].shape, k
        np.testing.assert_array_equal(v, inputs[k], err_msg=f"{name}: input {k}")
    got = mg.expected(p, inputs)
    assert sorted(got) == sorted(want)
    for k, w in want.items():
        g = got[k]
        assert g.dtype == w.dtype and g.shape == w.shape, k
        if w.dtype == np.float64:
            assert np.all(np.isfinite(w)), f"{name}: {k} not finite"
            scale = max(np.abs(w).max(), 1e-300)
            assert np.abs(g - w).max() <= 1e-12 * scale, f"{name}: {k}"
        else:
            np.testing.assert_array_equal(g, w, err_msg=f"{name}: output {k}")


def test_every_fixture_file_is_a_case():
    files = sorted(f[:-4] for f in os.listdir(mg.HERE) if f.endswith(".npz"))
    assert files == sorted(mg.CASES)
    total = sum(os.path.getsize(mg.path(n)) for n in files)
    assert total < 2 * 1024 * 1024, total


def test_golden_append_leaves_canary_outside_slots():
    """Independent of the oracle: the append fixtures change exactly the
    elements of their non-PAD slots, and every changed element holds the
    element of its token (bf16: the word itself)."""
    p, a, w = mg.load("append_gather_bf16_d64_bs16")
    kc, vc = w["key_cache"], w["value_cache"]
    bs, x = p["bs"], 8
    written_k = np.zeros(kc.shape, dtype=bool)
    written_v = np.zeros(vc.shape, dtype=bool)
    for t, s in enumerate(p["slots"]):
        if s < 0:
            continue
        blk, off = divmod(s, bs)
        for h in range(p["kvh"]):
            np.testing.assert_array_equal(kc[blk, h, :, off, :].reshape(-1), a["key"][t, h])
            np.testing.assert_array_equal(vc[blk, h, :, off], a["value"][t, h])
        written_k[blk, :, :, off, :] = True
        written_v[blk, :, :, off] = True
    assert np.all(kc[~written_k] == mg.CANARY16)
    assert np.all(vc[~written_v] == mg.CANARY16)
    # gather: sequence s, token i -> block bt[s, i // bs], offset i % bs
    cu = a["cu_seqlens_kv"]
    for s in range(len(cu) - 1):
        for i in range(int(cu[s + 1] - cu[s])):
            blk = a["block_tables"][s, i // bs]
            np.testing.assert_array_equal(w["gathered_key"][cu[s] + i],
                                          kc[blk, :, :, i % bs, :].reshape(p["kvh"], -1))
            np.testing.assert_array_equal(w["gathered_value"][cu[s] + i], vc[blk, :, :, i % bs])
    assert x * kc.shape[2] == p["d"]


def _value_row(p, vc, blk, kvh, off):
    """The dequantised V row of one token, as the query type rounds it."""
    code, kv = p["code"], p.get("kv", p["code"])
    if kv == mg.FP8:
        x = mg.orc.fp8_to_f32(vc[blk, kvh, :, off]).astype(np.float32) * np.float32(p["v_scale"])
        return mg.orc.to_f32(mg.orc.from_f32(x, code), code).astype(np.float64)
    return mg.orc.to_f32(vc[blk, kvh, :, off], code).astype(np.float64)


@pytest.mark.parametrize("name", sorted(n for n, c in mg.CASES.items() if c["op"] == "decode"))
def test_golden_decode_single_token_closed_form(name):
    """Independent of the oracle: a one-token context gives V[t0] / (1 + 1e-6)
    for every query head (softmax of one logit; the denominator term of the
    reference's paged kernel)."""
    p, a, w = mg.load(name)
    g = p["h"] // p["kvh"]
    seqs = [s for s, L in enumerate(p["lens"]) if L == 1]
    assert seqs
    for s in seqs:
        blk = a["block_tables"][s, 0]
        for h in range(p["h"]):
            want = _value_row(p, a["value_cache"], blk, h // g, 0) / (1 + 1e-6)
            np.testing.assert_allclose(w["out"][s, h], want, rtol=1e-12, atol=0)


@pytest.mark.parametrize("name", sorted(n for n, c in mg.CASES.items()
                                        if c["op"] == "prefill" and c["causal"]))
def test_golden_prefill_first_query_closed_form(name):
    """Independent of the oracle: in a causal prefill with no prior context
    the first query sees key 0 alone, so its output is V[0] (flash
    denominator, eps 0)."""
    p, a, w = mg.load(name)
    g = p["h"] // p["kvh"]
    cu = a["cu_seqlens_q"]
    seqs = [s for s, P in enumerate(p["prior"]) if P == 0]
    for s in seqs:
        blk = a["block_tables"][s, 0]
        for h in range(p["h"]):
            want = _value_row(p, a["value_cache"], blk, h // g, 0)
            np.testing.assert_allclose(w["out"][cu[s], h], want, rtol=1e-12, atol=0)
    # a sequence whose first query sees more than one key averages them:
    # the output lies inside the per-dimension hull of the visible V rows
    for s, P in enumerate(p["prior"]):
        n = P + 1
        rows = np.stack([_value_row(p, a["value_cache"], a["block_tables"][s, t // p["bs"]],
                                    0, t % p["bs"]) for t in range(n)])
        out = w["out"][cu[s], 0]
        assert np.all(out >= rows.min(0) - 1e-9) and np.all(out <= rows.max(0) + 1e-9)
