"""GPU parity of the device-side next-token selection and EOS state.

argmax_rows is checked bit-exactly (ids) against the oracle's restatement of
candle's argmax (first maximum; NaN only kept at element 0), on Qwen3-ASR's
vocabulary width and on odd widths, with planted ties, NaN and -inf rows
and strided rows. decode_consume_tokens is checked against the oracle over
multi-step runs, eagerly and replayed from a captured HIP graph (the
reference's decode loop runs inside graph replays, cuda_graph.rs:204-225)."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import TORCH, to_dev, to_host

pytestmark = pytest.mark.gpu

VOCAB = 151936  # Qwen3-ASR thinker vocabulary


def logits_case(rng, b, v, code):
    x = rng.standard_normal((b, v)).astype(np.float32) * 4
    for r in range(b):  # planted ties at the maximum
        m = x[r].max() + 1.0
        x[r, rng.choice(v, size=1 + r % 3, replace=False)] = m
    if b > 4:
        x[1, 0] = np.nan          # NaN at element 0: id 0
        x[2, 3 % v] = np.nan      # NaN elsewhere: ignored
        x[3, :] = -np.inf         # all -inf: id 0
        x[4, v // 2] = np.inf     # +inf wins
    return x if code == orc.F32 else orc.from_f32(x, code)


@pytest.mark.parametrize("code", [orc.BF16, orc.F16, orc.F32])
@pytest.mark.parametrize("v", [VOCAB, 1000, 37])
def test_argmax_rows_matches_oracle(device, code, v):
    rng = np.random.default_rng(v + code)
    b = 300 if v != VOCAB else 64
    x = logits_case(rng, b, v, code)
    got = vpa.argmax_token_ids_from_logits(to_dev(x, code, device))
    torch.cuda.synchronize()
    want = orc.argmax_rows(x, dtype=code)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_argmax_rows_strided_and_misaligned(device):
    """Rows that are a view into wider storage (row stride > vocab) and a
    start offset that breaks 16-byte alignment take the scalar path."""
    rng = np.random.default_rng(4)
    code = orc.BF16
    wide = logits_case(rng, 40, 1203, code)
    t = to_dev(wide, code, device)
    view = t[:, 1:1000]
    got = vpa.argmax_token_ids_from_logits(view)
    torch.cuda.synchronize()
    want = orc.argmax_rows(np.ascontiguousarray(wide[:, 1:1000]), dtype=code)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def run_steps(device, batch, steps, cap, eos, graph):
    rng = np.random.default_rng(batch + steps)
    v = 97
    st = vpa.DecodeTokenState(batch, cap, eos, device)
    pend = rng.integers(0, v, size=batch).astype(np.uint32)
    st.next_ids.copy_(torch.from_numpy(pend).to(device))
    logits_buf = torch.empty((batch, v), dtype=torch.bfloat16, device=device)
    # oracle state
    nid, fin = pend.copy(), np.zeros(batch, np.uint8)
    gen, glen = np.zeros((batch, cap), np.uint32), np.zeros(batch, np.uint32)

    def step():
        st.consume()
        st.select(logits_buf)

    g = None
    if graph:
        step()  # warm up, then restore the initial state before capturing
        torch.cuda.synchronize()
        st.next_ids.copy_(torch.from_numpy(pend).to(device))
        st.finished.zero_()
        st.gen_len.zero_()
        st.generated.zero_()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
    for s in range(steps):
        # a small vocabulary with heavy EOS ids so rows finish along the way
        lg = rng.standard_normal((batch, v)).astype(np.float32)
        lg[:, eos[0]] += rng.random(batch).astype(np.float32) * 2.5
        lw = orc.from_f32(lg, orc.BF16)
        logits_buf.copy_(to_dev(lw, orc.BF16, device))
        if graph:
            g.replay()
        else:
            step()
        torch.cuda.synchronize()
        inp, active = orc.decode_consume_tokens(nid, fin, gen, glen, eos, eos[0])
        nid = orc.argmax_rows(lw, dtype=orc.BF16)
        assert int(st.active_count.item()) == active, f"step {s}"
        np.testing.assert_array_equal(st.input_ids.cpu().numpy(), inp)
        np.testing.assert_array_equal(st.finished.cpu().numpy(), fin)
        np.testing.assert_array_equal(st.gen_len.cpu().numpy(), glen)
        np.testing.assert_array_equal(st.generated.cpu().numpy(), gen)
        np.testing.assert_array_equal(st.next_ids.cpu().numpy(), nid)


@pytest.mark.parametrize("graph", [False, True])
def test_decode_token_state_matches_oracle(device, graph):
    run_steps(device, batch=300, steps=12, cap=8, eos=[3, 11], graph=graph)


def test_consume_larger_batch_than_workgroup(device):
    run_steps(device, batch=2500, steps=3, cap=4, eos=[0], graph=False)
