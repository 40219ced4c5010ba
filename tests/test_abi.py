"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/vpa.h, and rejects bad arguments on the host before any
launch (so these calls never touch a device)."""

import ctypes
import os
import re

import pytest

from vpa import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names.update(re.findall(r"\b(vpa_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert "vpa_paged_attention" in names and "vpa_reshape_and_cache" in names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_version_and_empty_error():
    lib = _lib.load()
    assert lib.vpa_version().startswith(b"vpa")


def layout(kvh, d, bs, nb, dtype):
    ks = (ctypes.c_int64 * 5)()
    vs = (ctypes.c_int64 * 4)()
    rc = _lib.load().vpa_cache_layout(kvh, d, bs, nb, dtype, ks, vs)
    return rc, tuple(ks), tuple(vs)


def test_cache_layout_matches_reference_kat():
    # PagedKvCache::new(1, 2, 8, 4, 10, F32): 3 blocks, key [3,2,2,4,4],
    # value [3,2,8,4] (vasr-paged-attn/src/paged_kv_cache.rs:1091-1107)
    rc, ks, vs = layout(2, 8, 4, 3, _lib.DTYPE_F32)
    assert rc == 0
    assert ks == (3, 2, 2, 4, 4)
    assert vs == (3, 2, 8, 4)
    rc, ks, vs = layout(8, 128, 16, 100, _lib.DTYPE_BF16)
    assert rc == 0 and ks == (100, 8, 16, 16, 8) and vs == (100, 8, 128, 16)


@pytest.mark.parametrize("args,code,needle", [
    ((0, 8, 4, 3, 0), _lib.VPA_ERR_INVALID_ARGUMENT, "kv head"),
    ((2, 0, 4, 3, 0), _lib.VPA_ERR_INVALID_ARGUMENT, "head_dim"),
    ((2, 8, 0, 3, 0), _lib.VPA_ERR_INVALID_ARGUMENT, "block_size"),
    ((2, 8, 4, 0, 0), _lib.VPA_ERR_INVALID_ARGUMENT, "num_blocks"),
    ((2, 12, 4, 3, 2), _lib.VPA_ERR_INVALID_ARGUMENT, "divisible by key cache pack size"),
    ((2, 8, 4, 3, 9), _lib.VPA_ERR_UNSUPPORTED, "dtype"),
])
def test_cache_layout_rejects(args, code, needle):
    rc, _, _ = layout(*args)
    assert rc == code
    assert needle in _lib.load().vpa_last_error().decode()


FAKE = 1 << 20  # 16-byte aligned non-null host values standing in for device pointers


def rc_call(**over):
    args = dict(key=FAKE, value=FAKE, kts=1024, vts=1024, ks=None, vs=None, kc=FAKE, vc=FAKE,
                slots=FAKE, t=4, kvh=8, d=128, bs=16, nb=10, bstride=8 * 128 * 16,
                hstride=128 * 16, dtype=_lib.DTYPE_BF16, cdtype=_lib.DTYPE_BF16, stream=None)
    args.update(over)
    lib = _lib.load()
    rc = lib.vpa_reshape_and_cache(*args.values())
    return rc, lib.vpa_last_error().decode()


@pytest.mark.parametrize("over,code,needle", [
    (dict(dtype=_lib.DTYPE_F32), _lib.VPA_ERR_UNSUPPORTED, "differs"),
    (dict(dtype=7, cdtype=7), _lib.VPA_ERR_UNSUPPORTED, "dtype"),
    (dict(d=80), _lib.VPA_ERR_UNSUPPORTED, "no kernel"),
    (dict(bs=24), _lib.VPA_ERR_UNSUPPORTED, "no kernel"),
    (dict(hstride=100), _lib.VPA_ERR_INVALID_ARGUMENT, "strides"),
    (dict(bstride=128 * 16), _lib.VPA_ERR_INVALID_ARGUMENT, "strides"),
    (dict(kts=512), _lib.VPA_ERR_INVALID_ARGUMENT, "token stride"),
    (dict(slots=None), _lib.VPA_ERR_INVALID_ARGUMENT, "non-null"),
    (dict(kc=None), _lib.VPA_ERR_INVALID_ARGUMENT, "non-null"),
    (dict(key=FAKE + 2), _lib.VPA_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(t=-1), _lib.VPA_ERR_INVALID_ARGUMENT, "num_tokens"),
    (dict(nb=0), _lib.VPA_ERR_INVALID_ARGUMENT, "positive"),
    # one launch: groups of 16 tokens x 8 kv heads must stay below 2^24
    (dict(t=16 * (1 << 24) // 8), _lib.VPA_ERR_INVALID_ARGUMENT, "too many tokens"),
])
def test_reshape_and_cache_host_validation(over, code, needle):
    rc, msg = rc_call(**over)
    assert rc == code, msg
    assert needle in msg


def test_reshape_and_cache_zero_tokens_is_noop():
    rc, _ = rc_call(t=0, key=None, value=None, slots=None)
    assert rc == 0


def pa_call(**over):
    args = dict(out=FAKE, q=FAKE, ks=None, vs=None, kc=FAKE, vc=FAKE, bt=FAKE, bts=64, cl=FAKE,
                alibi=None, max_ctx=1024, scale=0.088, softcap=1.0, sinks=None, b=4, h=16, kvh=8,
                d=128, bs=16, nb=100, bstride=8 * 128 * 16, hstride=128 * 16,
                dtype=_lib.DTYPE_BF16, cdtype=_lib.DTYPE_BF16, ws=None, ws_bytes=0, stream=None)
    args.update(over)
    lib = _lib.load()
    rc = lib.vpa_paged_attention(*args.values())
    return rc, lib.vpa_last_error().decode()


@pytest.mark.parametrize("over,code,needle", [
    (dict(alibi=FAKE), _lib.VPA_ERR_UNSUPPORTED, "alibi"),
    (dict(sinks=FAKE), _lib.VPA_ERR_UNSUPPORTED, "sinks"),
    (dict(softcap=30.0), _lib.VPA_ERR_UNSUPPORTED, "softcapping"),
    (dict(h=12), _lib.VPA_ERR_INVALID_ARGUMENT, "multiple"),
    (dict(h=64), _lib.VPA_ERR_WORKSPACE, "workspace"),  # 8 per kv head: passes the shape checks
    (dict(h=24), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(bts=10), _lib.VPA_ERR_INVALID_ARGUMENT, "block_table_stride"),
    (dict(q=None), _lib.VPA_ERR_INVALID_ARGUMENT, "non-null"),
    (dict(cdtype=_lib.DTYPE_F16), _lib.VPA_ERR_UNSUPPORTED, "differs"),
    (dict(), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(ws=FAKE + 16, ws_bytes=1 << 30), _lib.VPA_ERR_INVALID_ARGUMENT, "256-byte"),
    (dict(max_ctx=1 << 30, bts=1 << 26), _lib.VPA_ERR_UNSUPPORTED, "max_context_len"),
    # one token past the longest context the split-K workspace holds
    # (2048 partitions of 128 tokens)
    (dict(max_ctx=262145, bts=1 << 15), _lib.VPA_ERR_UNSUPPORTED, "max_context_len"),
    # the longest context passes the size checks and then needs its workspace
    (dict(max_ctx=262144, bts=1 << 14), _lib.VPA_ERR_WORKSPACE, "workspace"),
])
def test_paged_attention_host_validation(over, code, needle):
    rc, msg = pa_call(**over)
    assert rc == code, msg
    assert needle in msg


def test_paged_attention_workspace_size():
    lib = _lib.load()
    # a single partition still needs the work list and queue
    small = lib.vpa_paged_attention_workspace_size(256, 16, 128, 128)
    assert 0 < small < 64 * 1024
    n = lib.vpa_paged_attention_workspace_size(256, 16, 128, 4096)
    rows = 256 * 16 * (4096 // 128)
    assert n >= rows * 128 * 4 + 2 * rows * 4 + small
    assert pa_call(b=0)[0] == 0  # empty batch: no launch, no workspace


def test_gather_host_validation():
    lib = _lib.load()
    rc = lib.vpa_gather_kv_cache(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, 4, FAKE, 2, 10, 8, 128,
                                 16, 100, 8 * 128 * 16, 128 * 16, _lib.DTYPE_BF16, _lib.DTYPE_F32,
                                 None)
    assert rc == _lib.VPA_ERR_UNSUPPORTED
    rc = lib.vpa_gather_kv_cache(None, FAKE, FAKE, FAKE, None, None, FAKE, 4, FAKE, 2, 10, 8, 128,
                                 16, 100, 8 * 128 * 16, 128 * 16, _lib.DTYPE_BF16,
                                 _lib.DTYPE_BF16, None)
    assert rc == _lib.VPA_ERR_INVALID_ARGUMENT
    rc = lib.vpa_gather_kv_cache(None, None, FAKE, FAKE, None, None, None, 4, None, 0, 0, 8, 128,
                                 16, 100, 8 * 128 * 16, 128 * 16, _lib.DTYPE_BF16,
                                 _lib.DTYPE_BF16, None)
    assert rc == 0
    # the grid's y (table column) and z (sequence) extents
    for bts, ns in ((65536, 2), (4, 65536)):
        rc = lib.vpa_gather_kv_cache(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, bts, FAKE, ns, 10,
                                     8, 128, 16, 100, 8 * 128 * 16, 128 * 16, _lib.DTYPE_BF16,
                                     _lib.DTYPE_BF16, None)
        assert rc == _lib.VPA_ERR_UNSUPPORTED and "65535" in lib.vpa_last_error().decode()


def pf_call(**over):
    args = dict(out=FAKE, q=FAKE, ks=None, vs=None, kc=FAKE, vc=FAKE, bt=FAKE, bts=64,
                cuq=FAKE, cl=FAKE, b=4, maxq=512, maxkv=1024, tq=2048, scale=0.088, eps=0.0,
                causal=1,
                h=16, kvh=8, d=128, bs=16, nb=100, bstride=8 * 128 * 16, hstride=128 * 16,
                dtype=_lib.DTYPE_BF16, cdtype=_lib.DTYPE_BF16, stream=None)
    args.update(over)
    lib = _lib.load()
    rc = lib.vpa_chunked_prefill_paged_attention(*args.values())
    return rc, lib.vpa_last_error().decode()


@pytest.mark.parametrize("over,code,needle", [
    (dict(d=80, bstride=8 * 80 * 16, hstride=80 * 16), _lib.VPA_ERR_UNSUPPORTED,
     "no kernel for dtype"),
    (dict(h=12), _lib.VPA_ERR_INVALID_ARGUMENT, "multiple"),
    (dict(dtype=5, cdtype=5), _lib.VPA_ERR_UNSUPPORTED, "query dtype"),
    (dict(cdtype=_lib.DTYPE_F16), _lib.VPA_ERR_UNSUPPORTED, "differs"),
    (dict(bts=10), _lib.VPA_ERR_INVALID_ARGUMENT, "block_table_stride"),
    (dict(cuq=None), _lib.VPA_ERR_INVALID_ARGUMENT, "non-null"),
    (dict(cl=None), _lib.VPA_ERR_INVALID_ARGUMENT, "non-null"),
    (dict(out=FAKE + 8), _lib.VPA_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(maxq=-1), _lib.VPA_ERR_INVALID_ARGUMENT, "bad sizes"),
    (dict(tq=-5), _lib.VPA_ERR_INVALID_ARGUMENT, "bad sizes"),
    (dict(hstride=100), _lib.VPA_ERR_INVALID_ARGUMENT, "strides"),
])
def test_prefill_host_validation(over, code, needle):
    rc, msg = pf_call(**over)
    assert rc == code, msg
    assert needle in msg


@pytest.mark.parametrize("over", [
    dict(dtype=_lib.DTYPE_F32, cdtype=_lib.DTYPE_F32, bstride=8 * 128 * 16 * 2,
         hstride=128 * 16 * 2),
    dict(dtype=_lib.DTYPE_F32, cdtype=_lib.DTYPE_FP8_E4M3, ks=FAKE, vs=FAKE,
         bstride=8 * 128 * 16, hstride=128 * 16),
    dict(d=96, bs=8, bstride=8 * 96 * 8, hstride=96 * 8),
    dict(cdtype=_lib.DTYPE_FP8_E4M3, ks=FAKE, vs=FAKE, d=96, bs=16, bstride=8 * 96 * 16,
         hstride=96 * 16),
    dict(h=64), dict(h=24), dict(h=128)])
def test_prefill_vector_kernel_configs_pass_validation(over):
    """The configurations the MFMA prefill is not built for go to the vector
    kernel: f32 queries over f32 and fp8 caches (the Metal prefill's `float`
    and `float, uint8_t` instances), the 16-bit / fp8 head-dim and block-size
    pairs without whole 1 KiB DMAs, and 8, 3 and 16 query heads per kv head.
    They pass every host check; an empty batch then returns before any
    launch."""
    rc, msg = pf_call(maxq=0, **over)
    assert rc == 0, msg


@pytest.mark.parametrize("d,bs,fp8", [(96, 16, False), (96, 32, False), (192, 8, False),
                                      (256, 8, False), (256, 32, False), (96, 32, True),
                                      (192, 16, True), (256, 32, True)])
def test_prefill_head_dims_pass_validation(d, bs, fp8):
    """head_dim 96 / 192 / 256 (the Metal prefill's set, varlen_prefill.rs:15)
    pass every host check; an empty batch then returns before any launch."""
    x = 16 if fp8 else 8
    over = dict(d=d, bs=bs, bstride=8 * d * bs, hstride=d * bs, maxq=0)
    if fp8:
        over.update(cdtype=FP8, ks=FAKE, vs=FAKE)
    assert (d * bs // x) % 64 == 0
    rc, msg = pf_call(**over)
    assert rc == 0, msg


@pytest.mark.parametrize("d,bs,dtype,ok", [
    (96, 8, _lib.DTYPE_BF16, True), (96, 16, _lib.DTYPE_BF16, True),
    (96, 8, _lib.DTYPE_F32, True), (192, 8, _lib.DTYPE_F16, True),
    (80, 16, _lib.DTYPE_BF16, False)])
def test_decode_head_dims_validation(d, bs, dtype, ok):
    """Decode at head_dim 96 and 192 passes validation at every block size
    (16-bit head_dim 96 at 8-token blocks, whose tile is not whole 1 KiB wave
    loads, on the chunked-prefill vector kernel); head_dim 80 is outside the
    reference's set."""
    rc, msg = pa_call(d=d, bs=bs, dtype=dtype, cdtype=dtype, bstride=8 * d * bs,
                      hstride=d * bs, b=0)
    if ok:
        assert rc == 0, msg
    else:
        assert rc == _lib.VPA_ERR_UNSUPPORTED, msg
        assert "head_dim" in msg


def test_prefill_empty_is_noop():
    assert pf_call(b=0, out=None, q=None)[0] == 0
    assert pf_call(maxq=0)[0] == 0
    assert pf_call(tq=0)[0] == 0


def plan_call(**over):
    args = dict(cl=FAKE, max_ctx=1024, bts=64, b=4, h=16, kvh=8, d=128, bs=16,
                dtype=_lib.DTYPE_BF16, ws=FAKE * 256, ws_bytes=1 << 30, stream=None)
    args.update(over)
    lib = _lib.load()
    rc = lib.vpa_paged_attention_plan(*args.values())
    return rc, lib.vpa_last_error().decode()


@pytest.mark.parametrize("over,code,needle", [
    (dict(ws=None), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(ws_bytes=16), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(ws=FAKE * 256 + 16), _lib.VPA_ERR_INVALID_ARGUMENT, "256-byte"),
    (dict(h=12), _lib.VPA_ERR_INVALID_ARGUMENT, "bad sizes"),
    (dict(d=80), _lib.VPA_ERR_UNSUPPORTED, "no decode kernel"),
    (dict(cl=None), _lib.VPA_ERR_INVALID_ARGUMENT, "non-null"),
    (dict(bts=10), _lib.VPA_ERR_INVALID_ARGUMENT, "block_table_stride"),
    (dict(b=70000), _lib.VPA_ERR_UNSUPPORTED, "num_seqs"),
])
def test_paged_attention_plan_host_validation(over, code, needle):
    rc, msg = plan_call(**over)
    assert rc == code, msg
    assert needle in msg


def test_paged_attention_planned_validates_like_paged_attention():
    lib = _lib.load()
    for over in (dict(alibi=FAKE), dict(softcap=2.0), dict(), dict(h=12)):
        args = dict(out=FAKE, q=FAKE, ks=None, vs=None, kc=FAKE, vc=FAKE, bt=FAKE, bts=64, cl=FAKE,
                    alibi=None, max_ctx=1024, scale=0.088, softcap=1.0, sinks=None, b=4, h=16,
                    kvh=8, d=128, bs=16, nb=100, bstride=8 * 128 * 16, hstride=128 * 16,
                    dtype=_lib.DTYPE_BF16, cdtype=_lib.DTYPE_BF16, ws=None, ws_bytes=0,
                    stream=None)
        args.update(over)
        rc_a = lib.vpa_paged_attention(*args.values())
        msg_a = lib.vpa_last_error().decode()
        rc_b = lib.vpa_paged_attention_planned(*args.values())
        msg_b = lib.vpa_last_error().decode()
        assert rc_a == rc_b != 0
        assert msg_b.replace("paged_attention_planned", "paged_attention") == msg_a


# ---- fp8 (E4M3FN) caches -------------------------------------------------------

FP8 = _lib.DTYPE_FP8_E4M3
F8_STRIDES = dict(bstride=8 * 128 * 16, hstride=128 * 16)  # in bytes = elements


def test_cache_layout_fp8_packs_16():
    rc, ks, vs = layout(8, 128, 16, 100, FP8)
    assert rc == 0 and ks == (100, 8, 8, 16, 16) and vs == (100, 8, 128, 16)
    rc, _, _ = layout(8, 72, 16, 100, FP8)
    assert rc == _lib.VPA_ERR_INVALID_ARGUMENT  # 72 is not a multiple of 16


@pytest.mark.parametrize("over,code,needle", [
    (dict(cdtype=FP8, **F8_STRIDES), _lib.VPA_ERR_INVALID_ARGUMENT, "k_scale and v_scale"),
    (dict(cdtype=FP8, ks=FAKE, **F8_STRIDES), _lib.VPA_ERR_INVALID_ARGUMENT, "k_scale and v_scale"),
    (dict(cdtype=FP8, ks=FAKE + 2, vs=FAKE, **F8_STRIDES), _lib.VPA_ERR_INVALID_ARGUMENT,
     "4-byte aligned"),
    (dict(dtype=FP8, cdtype=FP8, ks=FAKE, vs=FAKE, **F8_STRIDES), _lib.VPA_ERR_UNSUPPORTED,
     "input dtype"),
])
def test_reshape_and_cache_fp8_validation(over, code, needle):
    rc, msg = rc_call(**over)
    assert rc == code, msg
    assert needle in msg


@pytest.mark.parametrize("dtype", [_lib.DTYPE_F32, _lib.DTYPE_F16, _lib.DTYPE_BF16])
def test_reshape_and_cache_fp8_accepts_every_float_input(dtype):
    # validation passes up to the launch, which a GPU-less host cannot do:
    # only the HIP status may fail (never an argument or support error)
    rc, msg = rc_call(dtype=dtype, cdtype=FP8, ks=FAKE, vs=FAKE, t=0, **F8_STRIDES)
    assert rc == 0, msg


@pytest.mark.parametrize("over,code,needle", [
    (dict(cdtype=FP8, **F8_STRIDES), _lib.VPA_ERR_INVALID_ARGUMENT, "k_scale and v_scale"),
    # f32 queries over fp8 caches: the generic split-K kernel, tiles of up to
    # 6 KiB at 16- and 32-token blocks
    (dict(dtype=_lib.DTYPE_F32, cdtype=FP8, ks=FAKE, vs=FAKE, **F8_STRIDES),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(dtype=_lib.DTYPE_F32, cdtype=FP8, ks=FAKE, vs=FAKE, d=192, bs=32,
          bstride=8 * 192 * 32, hstride=192 * 32), _lib.VPA_ERR_WORKSPACE, "workspace"),
    # the pairs no decode kernel takes run on the chunked-prefill vector
    # kernel: validation passes up to the workspace check
    (dict(dtype=_lib.DTYPE_F32, cdtype=FP8, ks=FAKE, vs=FAKE, d=256, bs=32,
          bstride=8 * 256 * 32, hstride=256 * 32), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(dtype=_lib.DTYPE_F32, cdtype=FP8, ks=FAKE, vs=FAKE, bs=8, bts=128, bstride=8 * 128 * 8,
          hstride=128 * 8), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=64, bs=8, bts=128, bstride=8 * 64 * 8,
          hstride=64 * 8), _lib.VPA_ERR_WORKSPACE, "workspace"),
    # head dims 192 and 256 at 32-token blocks under 16-bit queries: the
    # generic kernel, validation passes up to the workspace check
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=256, bs=32, bstride=8 * 256 * 32, hstride=256 * 32),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=192, bs=32, bstride=8 * 192 * 32, hstride=192 * 32),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=192, bs=8, bts=128, bstride=8 * 192 * 8,
          hstride=192 * 8), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=96, bs=16, bstride=8 * 96 * 16, hstride=96 * 16),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=80, bs=16, bstride=8 * 80 * 16, hstride=80 * 16),
     _lib.VPA_ERR_UNSUPPORTED, "no kernel"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, **F8_STRIDES), _lib.VPA_ERR_WORKSPACE, "workspace"),
    # head dims 96 / 192 / 256 on the rows kernel: validation passes up to
    # the workspace check
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=96, bs=32, bstride=8 * 96 * 32, hstride=96 * 32),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=192, bs=16, bstride=8 * 192 * 16, hstride=192 * 16),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=256, bs=8, bts=128, bstride=8 * 256 * 8,
          hstride=256 * 8), _lib.VPA_ERR_WORKSPACE, "workspace"),
    (dict(cdtype=FP8, ks=FAKE, vs=FAKE, d=256, bs=16, bstride=8 * 256 * 16, hstride=256 * 16),
     _lib.VPA_ERR_WORKSPACE, "workspace"),
])
def test_paged_attention_fp8_validation(over, code, needle):
    rc, msg = pa_call(**over)
    assert rc == code, msg
    assert needle in msg


def test_gather_and_prefill_fp8_validation():
    lib = _lib.load()
    args = [FAKE, FAKE, FAKE, FAKE, None, None, FAKE, 4, FAKE, 2, 10, 8, 128, 16, 100,
            8 * 128 * 16, 128 * 16, FP8, _lib.DTYPE_BF16, None]
    assert lib.vpa_gather_kv_cache(*args) == _lib.VPA_ERR_INVALID_ARGUMENT  # no scales
    assert "k_scale" in lib.vpa_last_error().decode()
    args[4], args[5], args[17], args[18] = FAKE, FAKE, _lib.DTYPE_BF16, _lib.DTYPE_F32
    assert lib.vpa_gather_kv_cache(*args) == _lib.VPA_ERR_UNSUPPORTED  # 16-bit cache -> other
    args[17], args[18], args[9] = FP8, FP8, 0  # fp8 -> fp8 (raw bytes), empty batch
    assert lib.vpa_gather_kv_cache(*args) == 0, lib.vpa_last_error().decode()
    # prefill over an fp8 cache: validation only (no device here)
    rc, msg = pf_call(cdtype=FP8, **F8_STRIDES)
    assert rc == _lib.VPA_ERR_INVALID_ARGUMENT and "k_scale" in msg, msg
    rc, msg = pf_call(cdtype=FP8, ks=FAKE, vs=FAKE, dtype=_lib.DTYPE_F32, maxq=0, **F8_STRIDES)
    assert rc == 0, msg
    rc, msg = pf_call(cdtype=FP8, ks=FAKE, vs=FAKE, d=64, bs=8, bstride=8 * 64 * 8,
                      hstride=64 * 8, maxq=0)
    assert rc == 0, msg
    # fp8 at 8-token blocks: head_dim 128 (decode and prefill) and 256 (prefill)
    rc, msg = pf_call(cdtype=FP8, ks=FAKE, vs=FAKE, bs=8, bstride=8 * 128 * 8, hstride=128 * 8,
                      maxq=0)
    assert rc == 0, msg
    rc, msg = pf_call(cdtype=FP8, ks=FAKE, vs=FAKE, d=256, bs=8, bstride=8 * 256 * 8,
                      hstride=256 * 8, maxq=0)
    assert rc == 0, msg
    rc, msg = pa_call(cdtype=FP8, ks=FAKE, vs=FAKE, bs=8, bstride=8 * 128 * 8, hstride=128 * 8,
                      b=0)
    assert rc == 0, msg


def test_paged_cache_read_validation():
    lib = _lib.load()

    def call(**over):
        a = dict(kc=FAKE, vc=FAKE, bt=FAKE, bts=64, max_ctx=1024, b=4, h=16, kvh=8, d=128, bs=16,
                 nb=100, bstride=8 * 128 * 16, hstride=128 * 16, cdt=_lib.DTYPE_BF16, ws=None,
                 ws_bytes=0, magic=0, sink=FAKE, stream=None)
        a.update(over)
        return lib.vpa_paged_cache_read(*a.values()), lib.vpa_last_error().decode()

    rc, msg = call()
    assert rc == _lib.VPA_ERR_WORKSPACE and "workspace" in msg, msg
    rc, msg = call(cdt=_lib.DTYPE_F32, bstride=8 * 128 * 16, hstride=128 * 16)
    assert rc == _lib.VPA_ERR_UNSUPPORTED, msg
    rc, msg = call(bts=10)
    assert rc == _lib.VPA_ERR_INVALID_ARGUMENT and "block_table_stride" in msg, msg
    rc, msg = call(sink=None)
    assert rc == _lib.VPA_ERR_INVALID_ARGUMENT and "sink" in msg, msg
    assert call(b=0)[0] == 0


def test_noalloc_validates_before_touching_the_device():
    """vpa_paged_attention_noalloc runs every argument check of
    vpa_paged_attention (same codes and messages) and its own scratch-size
    check before it looks up its scratch on the device (there is none here)."""
    lib = _lib.load()
    for over in (dict(alibi=FAKE), dict(softcap=2.0), dict(h=12), dict(bts=10)):
        args = dict(out=FAKE, q=FAKE, ks=None, vs=None, kc=FAKE, vc=FAKE, bt=FAKE, bts=64, cl=FAKE,
                    alibi=None, max_ctx=1024, scale=0.088, softcap=1.0, sinks=None, b=4, h=16,
                    kvh=8, d=128, bs=16, nb=100, bstride=8 * 128 * 16, hstride=128 * 16,
                    dtype=_lib.DTYPE_BF16, cdtype=_lib.DTYPE_BF16)
        args.update(over)
        rc_a = lib.vpa_paged_attention(*args.values(), None, 0, None)
        msg_a = lib.vpa_last_error().decode()
        rc_b = lib.vpa_paged_attention_noalloc(*args.values(), None)
        msg_b = lib.vpa_last_error().decode()
        assert rc_a == rc_b != 0 and rc_a != _lib.VPA_ERR_WORKSPACE, msg_a
        assert msg_b.replace("paged_attention_noalloc", "paged_attention") == msg_a
    # 4096 sequences of 16384 tokens: 335 MB of partial rows > the 64 MiB scratch
    rc = lib.vpa_paged_attention_noalloc(FAKE, FAKE, None, None, FAKE, FAKE, FAKE, 1024, FAKE,
                                         None, 16384, 0.088, 1.0, None, 4096, 16, 8, 128, 16,
                                         100, 8 * 128 * 16, 128 * 16, _lib.DTYPE_BF16,
                                         _lib.DTYPE_BF16, None)
    assert rc == _lib.VPA_ERR_WORKSPACE and "static scratch" in lib.vpa_last_error().decode()


# ---- fused append + decode -------------------------------------------------------

def fused_args(**over):
    args = dict(out=FAKE, q=FAKE, k=FAKE, v=FAKE, kts=8 * 128, vts=8 * 128, ks=None, vs=None,
                kc=FAKE, vc=FAKE, bt=FAKE, bts=64, cl=FAKE, max_ctx=1024, scale=0.088, b=4, h=16,
                kvh=8, d=128, bs=16, nb=100, bstride=8 * 128 * 16, hstride=128 * 16,
                dtype=_lib.DTYPE_BF16, cdtype=_lib.DTYPE_BF16, ws=None, ws_bytes=0, stream=None)
    args.update(over)
    return args


def fused_call(**over):
    lib = _lib.load()
    rc = lib.vpa_reshape_and_cache_paged_attention(*fused_args(**over).values())
    return rc, lib.vpa_last_error().decode()


@pytest.mark.parametrize("over,code,needle", [
    (dict(k=None), _lib.VPA_ERR_INVALID_ARGUMENT, "key and value"),
    (dict(vts=100), _lib.VPA_ERR_INVALID_ARGUMENT, "token stride"),
    (dict(k=FAKE + 2), _lib.VPA_ERR_INVALID_ARGUMENT, "16-byte aligned"),
    (dict(h=12), _lib.VPA_ERR_INVALID_ARGUMENT, "multiple"),
    (dict(bts=10), _lib.VPA_ERR_INVALID_ARGUMENT, "block_table_stride"),
    (dict(cdtype=_lib.DTYPE_FP8_E4M3), _lib.VPA_ERR_INVALID_ARGUMENT, "k_scale"),
    (dict(dtype=_lib.DTYPE_F32), _lib.VPA_ERR_UNSUPPORTED, "differs"),
    (dict(ws_bytes=0, max_ctx=4096, bts=256), _lib.VPA_ERR_WORKSPACE, "workspace"),
])
def test_fused_append_decode_host_validation(over, code, needle):
    """vpa_reshape_and_cache_paged_attention: every check of the two calls it
    stands for runs on the host, with the entry point's name."""
    rc, msg = fused_call(**over)
    assert rc == code, msg
    assert needle in msg, msg
    assert msg.startswith("reshape_and_cache_paged_attention")


def test_fused_append_decode_planned_validates_alike():
    lib = _lib.load()
    for over in (dict(dtype=_lib.DTYPE_F32), dict(k=None), dict(h=12), dict(bts=10)):
        args = fused_args(**over)
        rc_a = lib.vpa_reshape_and_cache_paged_attention(*args.values())
        msg_a = lib.vpa_last_error().decode()
        rc_b = lib.vpa_reshape_and_cache_paged_attention_planned(*args.values())
        msg_b = lib.vpa_last_error().decode()
        assert rc_a == rc_b != 0
        assert msg_b.replace("_planned", "") == msg_a
    assert fused_call(b=0)[0] == 0
