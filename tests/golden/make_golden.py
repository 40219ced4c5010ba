"""TEST INFRASTRUCTURE ONLY — writes the golden fixtures of this directory.

Each fixture is a small seeded case of one op on the hot path: its inputs
and the expected outputs computed by the CPU oracle (``oracle/``), saved as
``<name>.npz`` (plain arrays, loadable with ``allow_pickle=False``; the
case's parameters are a JSON string under ``meta``). The oracle restates
the reference's semantics (file:line citations in ``oracle/vpa_oracle.c``):
paged cache layout and slot rule (``paged_kv_cache.rs:7, 74-103, 263-294``),
GQA decode attention (``thinker_text.rs:1126-1139``, ``attention.rs:12-21,
243-286``), cached-causal chunked prefill (``attention.rs:78-149``; the
Metal kernel's ``+1e-6`` denominator, ``prefill_paged_attn.metal:1300``),
fp8 E4M3FN caches with scales (``.metal:698-769``), argmax
(``generation.rs:443-460``).

``tests/test_golden.py`` (CPU) recomputes every expected output from the
stored inputs with the oracle, so a change of the oracle shows against the
committed vectors; ``tests/test_gpu_golden.py`` runs the HIP library on the
stored inputs and compares with the stored outputs (attention within the
acceptance tolerance, appends, gathers and argmax bit for bit).

Run ``python tests/golden/make_golden.py`` from the repository root to
rewrite the fixtures.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

F32, F16, BF16, FP8 = orc.F32, orc.F16, orc.BF16, orc.FP8

# Canary words the append cases start their caches from: every element the
# append does not write must keep it.
CANARY16 = 0x3C5A
CANARY8 = 0x5A

CASES = {
    # decode: paged_attention over a shuffled pool, ragged lengths across
    # block and partition edges
    "decode_f32_gqa2_d64_bs16": dict(op="decode", code=F32, h=4, kvh=2, d=64, bs=16,
                                     lens=[1, 16, 17, 100], seed=11),
    "decode_bf16_gqa2_d128_bs16": dict(op="decode", code=BF16, h=2, kvh=1, d=128, bs=16,
                                       lens=[1, 15, 16, 33, 250], seed=12),
    "decode_f16_gqa4_d128_bs32": dict(op="decode", code=F16, h=4, kvh=1, d=128, bs=32,
                                      lens=[1, 31, 33, 150], seed=13),
    "decode_fp8_bf16q_d128_bs16": dict(op="decode", code=BF16, kv=FP8, h=2, kvh=1, d=128, bs=16,
                                       lens=[1, 17, 200], k_scale=0.7, v_scale=1.3, seed=14),
    # chunked prefill: new tokens over prior context in the paged cache
    "prefill_bf16_causal_d128_bs16": dict(op="prefill", code=BF16, h=2, kvh=1, d=128, bs=16,
                                          qlens=[5, 40, 1], prior=[0, 50, 32], causal=True,
                                          eps=0.0, seed=15),
    "prefill_f16_noncausal_eps_d64_bs8": dict(op="prefill", code=F16, h=2, kvh=2, d=64, bs=8,
                                              qlens=[3, 20], prior=[7, 25], causal=False,
                                              eps=1e-6, seed=16),
    "prefill_fp8_causal_d128_bs16": dict(op="prefill", code=BF16, kv=FP8, h=2, kvh=1, d=128,
                                         bs=16, qlens=[7, 33], prior=[0, 37], causal=True,
                                         eps=0.0, k_scale=0.5, v_scale=2.0, seed=17),
    # reshape_and_cache into canary-filled caches (a PAD slot, block edges),
    # then gather_kv_cache of two sequences
    "append_gather_bf16_d64_bs16": dict(op="append_gather", code=BF16, kvh=2, d=64, bs=16, nb=4,
                                        slots=[3, -1, 17, 31, 32, 63], bt=[[1, 2], [0, 3]],
                                        kv_lens=[20, 32], seed=18),
    "append_gather_fp8_d128_bs16": dict(op="append_gather", code=BF16, kv=FP8, kvh=1, d=128,
                                        bs=16, nb=3, slots=[5, -1, 16, 47], bt=[[0, 1], [2, 0]],
                                        kv_lens=[20, 16], k_scale=0.37, v_scale=3.1, seed=19),
    # argmax over rows with planted ties, NaN and infinities
    "argmax_bf16": dict(op="argmax", code=BF16, rows=7, vocab=1000, seed=20),
    "argmax_f32": dict(op="argmax", code=F32, rows=7, vocab=777, seed=21),
}


def _words(rng, shape, code, mult=1.0):
    return orc.from_f32((rng.standard_normal(shape) * mult).astype(np.float32), code)


def _fp8_bytes(rng, shape):
    return orc.fp8_from_f32((rng.standard_normal(shape) * 2).astype(np.float32))


def _cache(rng, nb, kvh, d, bs, code, kv):
    if kv == FP8:
        return _fp8_bytes(rng, (nb, kvh, d // 16, bs, 16)), _fp8_bytes(rng, (nb, kvh, d, bs))
    x = 4 if code == F32 else 8
    return _words(rng, (nb, kvh, d // x, bs, x), code), _words(rng, (nb, kvh, d, bs), code)


def _tables(rng, lens, nb, bs):
    need = [(max(int(L), 1) + bs - 1) // bs for L in lens]
    ids = rng.permutation(np.arange(1, nb))
    bt = np.zeros((len(lens), max(need)), dtype=np.uint32)
    off = 0
    for s, n in enumerate(need):
        bt[s, :n] = ids[off:off + n]
        off += n
    return bt


def make_inputs(p: dict) -> dict:
    """The seeded inputs of case ``p``."""
    rng = np.random.default_rng(p["seed"])
    code, kv = p["code"], p.get("kv", p["code"])
    if p["op"] == "decode":
        lens = np.asarray(p["lens"], dtype=np.uint32)
        nb = int(sum((int(L) + p["bs"] - 1) // p["bs"] for L in lens)) + 3
        kc, vc = _cache(rng, nb, p["kvh"], p["d"], p["bs"], code, kv)
        bt = _tables(rng, lens, nb, p["bs"])
        q = _words(rng, (len(lens), p["h"], p["d"]), code)
        return dict(q=q, key_cache=kc, value_cache=vc, block_tables=bt, context_lens=lens)
    if p["op"] == "prefill":
        qlens = np.asarray(p["qlens"], dtype=np.int64)
        lens = (np.asarray(p["prior"], dtype=np.int64) + qlens).astype(np.uint32)
        nb = int(sum((int(L) + p["bs"] - 1) // p["bs"] for L in lens)) + 3
        kc, vc = _cache(rng, nb, p["kvh"], p["d"], p["bs"], code, kv)
        bt = _tables(rng, lens, nb, p["bs"])
        q = _words(rng, (int(qlens.sum()), p["h"], p["d"]), code)
        cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
        return dict(q=q, key_cache=kc, value_cache=vc, block_tables=bt, context_lens=lens,
                    cu_seqlens_q=cu)
    if p["op"] == "append_gather":
        t = len(p["slots"])
        mult = 20.0 if kv == FP8 else 1.0  # fp8: saturating and subnormal values too
        key = _words(rng, (t, p["kvh"], p["d"]), code, mult)
        value = _words(rng, (t, p["kvh"], p["d"]), code, mult)
        return dict(key=key, value=value, slot_mapping=np.asarray(p["slots"], dtype=np.int64),
                    block_tables=np.asarray(p["bt"], dtype=np.uint32),
                    cu_seqlens_kv=np.concatenate([[0], np.cumsum(p["kv_lens"])]).astype(np.uint32))
    if p["op"] == "argmax":
        x = rng.standard_normal((p["rows"], p["vocab"])).astype(np.float32)
        v = p["vocab"]
        x[1, [7, v // 2]] = 50.0                   # tie: the first index wins
        x[2, 0] = np.nan                           # NaN at element 0
        x[3, [3, v - 2]] = np.nan                  # NaN inside the row
        x[3, 11] = 60.0
        x[4, :] = -np.inf                          # every element -inf
        x[5, [9, v - 1]] = np.inf                  # +inf twice
        x[6, v - 1] = 70.0                         # maximum at the last element
        return dict(logits=orc.from_f32(x, code))
    raise ValueError(p["op"])


def expected(p: dict, a: dict) -> dict:
    """The oracle's outputs for case ``p`` over inputs ``a``."""
    code, kv = p["code"], p.get("kv", p["code"])
    fp8 = kv == FP8
    ks, vs = p.get("k_scale", 1.0), p.get("v_scale", 1.0)
    scale = p["d"] ** -0.5 if "d" in p else None
    if p["op"] == "decode":
        out = orc.paged_attention(a["q"], a["key_cache"], a["value_cache"], a["block_tables"],
                                  a["context_lens"], int(a["context_lens"].max()), scale,
                                  dtype=code, kv_dtype=FP8 if fp8 else None, k_scale=ks,
                                  v_scale=vs)
        return dict(out=out)
    if p["op"] == "prefill":
        out = orc.prefill_attention(a["q"], a["key_cache"], a["value_cache"], a["block_tables"],
                                    a["context_lens"], a["cu_seqlens_q"], scale,
                                    causal=p["causal"], dtype=code, eps=p["eps"],
                                    kv_dtype=FP8 if fp8 else None, k_scale=ks, v_scale=vs)
        return dict(out=out)
    if p["op"] == "append_gather":
        nb, kvh, d, bs = p["nb"], p["kvh"], p["d"], p["bs"]
        if fp8:
            kc = np.full((nb, kvh, d // 16, bs, 16), CANARY8, dtype=np.uint8)
            vc = np.full((nb, kvh, d, bs), CANARY8, dtype=np.uint8)
            orc.reshape_and_cache_fp8(a["key"], a["value"], kc, vc, a["slot_mapping"], code,
                                      ks, vs)
            gk, gv = orc.gather_kv_cache_fp8(kc, vc, a["block_tables"], a["cu_seqlens_kv"],
                                             code, ks, vs)
        else:
            x = 4 if code == F32 else 8
            kc = np.full((nb, kvh, d // x, bs, x), CANARY16, dtype=np.uint16)
            vc = np.full((nb, kvh, d, bs), CANARY16, dtype=np.uint16)
            orc.reshape_and_cache(a["key"], a["value"], kc, vc, a["slot_mapping"], dtype=code)
            gk, gv = orc.gather_kv_cache(kc, vc, a["block_tables"], a["cu_seqlens_kv"],
                                         dtype=code)
        return dict(key_cache=kc, value_cache=vc, gathered_key=gk, gathered_value=gv)
    if p["op"] == "argmax":
        return dict(ids=orc.argmax_rows(a["logits"], dtype=code))
    raise ValueError(p["op"])


def path(name: str) -> str:
    return os.path.join(HERE, f"{name}.npz")


def load(name: str):
    """(params, inputs, expected) of a committed fixture."""
    with np.load(path(name), allow_pickle=False) as z:
        p = json.loads(str(z["meta"]))
        inputs = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
        want = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    return p, inputs, want


def main() -> None:
    for name, p in CASES.items():
        a = make_inputs(p)
        e = expected(p, a)
        arrays = {f"in_{k}": v for k, v in a.items()}
        arrays.update({f"out_{k}": v for k, v in e.items()})
        np.savez_compressed(path(name), meta=np.array(json.dumps(p, sort_keys=True)), **arrays)
        print(f"{name}: {os.path.getsize(path(name))} bytes")


if __name__ == "__main__":
    main()
