"""The HIP library on the committed golden fixtures (tests/golden/*.npz).

Each case's stored inputs go through the C ABI (vpa ops) and the results are
compared with the stored outputs: attention within the acceptance tolerance
(rel 1e-5 f32, 2e-2 bf16/f16, tests/_util.assert_attention_close) of the
fp64 outputs; reshape_and_cache (whole caches, canary included),
gather_kv_cache and argmax bit for bit. No oracle runs here: the expected
values are the committed ones."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import TORCH, assert_attention_close, i64, to_dev, to_host, u32
from tests.golden import make_golden as mg

pytestmark = pytest.mark.gpu


def _f8(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device).view(
        torch.float8_e4m3fn)


def _f8_host(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def _scalar(v, device):
    return torch.tensor([v], dtype=torch.float32, device=device)


def _caches(p, kc, vc, device):
    if p.get("kv") == mg.FP8:
        return (_f8(kc, device), _f8(vc, device), _scalar(p["k_scale"], device),
                _scalar(p["v_scale"], device))
    return to_dev(kc, p["code"], device), to_dev(vc, p["code"], device), None, None


def _same_words(got, want, code, what):
    """Bit equality; NaN payloads need only agree on being NaN."""
    if code == orc.F32 or got.dtype == np.uint8:
        np.testing.assert_array_equal(got, want, err_msg=what)
        return
    gf, wf = orc.to_f32(got, code), orc.to_f32(want, code)
    assert np.array_equal(np.isnan(gf), np.isnan(wf)), what
    fin = ~np.isnan(wf)
    np.testing.assert_array_equal(got[fin], want[fin], err_msg=what)


@pytest.mark.parametrize("name", sorted(mg.CASES))
def test_hip_matches_golden(device, name):
    p, a, want = mg.load(name)
    code = p["code"]
    print(f"golden case {name}", flush=True)
    if p["op"] == "decode":
        kc, vc, ks, vs = _caches(p, a["key_cache"], a["value_cache"], device)
        out = vpa.paged_attention(to_dev(a["q"], code, device), ks, vs, kc, vc,
                                  u32(a["block_tables"], device), u32(a["context_lens"], device),
                                  None, int(a["context_lens"].max()), p["d"] ** -0.5, 1.0, None)
        torch.cuda.synchronize()
        assert_attention_close(orc.to_f32(to_host(out), code), want["out"], code, name)
    elif p["op"] == "prefill":
        kc, vc, ks, vs = _caches(p, a["key_cache"], a["value_cache"], device)
        out = vpa.paged_attention_varlen_prefill(
            to_dev(a["q"], code, device), kc, vc, u32(a["block_tables"], device),
            u32(a["context_lens"], device), u32(a["cu_seqlens_q"], device), ks, vs,
            p["d"] ** -0.5, 1.0, causal=p["causal"], denom_eps=p["eps"])
        torch.cuda.synchronize()
        assert_attention_close(orc.to_f32(to_host(out), code), want["out"], code, name)
    elif p["op"] == "append_gather":
        fp8 = p.get("kv") == mg.FP8
        canary = mg.CANARY8 if fp8 else mg.CANARY16
        kc0 = np.full(want["key_cache"].shape, canary, dtype=want["key_cache"].dtype)
        vc0 = np.full(want["value_cache"].shape, canary, dtype=want["value_cache"].dtype)
        kc, vc, ks, vs = _caches(p, kc0, vc0, device)
        vpa.reshape_and_cache(to_dev(a["key"], code, device), to_dev(a["value"], code, device),
                              ks, vs, kc, vc, i64(a["slot_mapping"], device))
        gk, gv = vpa.gather_kv_cache(kc, vc, ks, vs, u32(a["block_tables"], device),
                                     u32(a["cu_seqlens_kv"], device), TORCH[code])
        torch.cuda.synchronize()
        host = _f8_host if fp8 else to_host
        np.testing.assert_array_equal(host(kc), want["key_cache"], err_msg=f"{name} key cache")
        np.testing.assert_array_equal(host(vc), want["value_cache"],
                                      err_msg=f"{name} value cache")
        _same_words(to_host(gk), want["gathered_key"], code, f"{name} gathered key")
        _same_words(to_host(gv), want["gathered_value"], code, f"{name} gathered value")
    elif p["op"] == "argmax":
        ids = vpa.argmax_token_ids_from_logits(to_dev(a["logits"], code, device))
        np.testing.assert_array_equal(ids.cpu().numpy(), want["ids"], err_msg=name)
    else:
        raise AssertionError(p["op"])
