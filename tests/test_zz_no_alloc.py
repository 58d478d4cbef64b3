"""pe_decode_attn_noalloc (the decode attention with its split records in the library's own
scratch array) against pe_decode_attn (caller workspace), through the C ABI: the same kernels,
so the outputs must be bit-identical, on two calls in a row, the second smaller than the first
(the scratch keeps the first call's records)."""

import ctypes

import pytest
import torch

from pico_hip import _lib
from pico_hip._lib import lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(seed, n_head, n_kv, hd, capacity, S, layout):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(n_head, hd, generator=g).cuda()
    k = torch.randn(n_kv, capacity, hd, generator=g).cuda()
    v = torch.randn(n_kv, capacity, hd, generator=g).cuda()
    S_dev = torch.tensor([S - 1], dtype=torch.int64, device="cuda")
    return q, k, v, S_dev


def _run_ws(q, k, v, S_dev, layout):
    n_head, hd = q.shape
    n_kv, capacity = k.shape[0], k.shape[1]
    nbytes = lib.pe_decode_attn_workspace_bytes(n_head, n_kv, hd, capacity)
    ws = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device="cuda")
    out = torch.empty(n_head, hd, device="cuda")
    _lib.check(lib.pe_decode_attn(_ptr(q), _ptr(k), _ptr(v), n_head, n_kv, hd, capacity,
                                  _ptr(S_dev), 2, 1, 0.125 if hd == 64 else hd ** -0.5, 1,
                                  _ptr(out), _ptr(ws), nbytes, layout, _stream()), "pe_decode_attn")
    return out


def _run_noalloc(q, k, v, S_dev, layout):
    n_head, hd = q.shape
    n_kv, capacity = k.shape[0], k.shape[1]
    out = torch.full((n_head, hd), float("nan"), device="cuda")
    _lib.check(lib.pe_decode_attn_noalloc(_ptr(q), _ptr(k), _ptr(v), n_head, n_kv, hd, capacity,
                                          _ptr(S_dev), 2, 1, 0.125 if hd == 64 else hd ** -0.5, 1,
                                          _ptr(out), layout, _stream()), "pe_decode_attn_noalloc")
    return out


@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 14, 2), (128, 28, 4)])
def test_noalloc_matches_workspace_entry_point_twice_shrinking(hd, n_head, n_kv):
    # split path (capacity > 256); the second call is smaller (fewer splits, shorter S)
    first = _case(1, n_head, n_kv, hd, 8192, 7000, 0)
    second = _case(2, n_head, n_kv, hd, 1024, 600, 0)
    outs = []
    for q, k, v, S_dev in (first, second):
        a = _run_noalloc(q, k, v, S_dev, 2)
        b = _run_ws(q, k, v, S_dev, 2)
        torch.cuda.synchronize()
        assert torch.isfinite(a).all()
        assert torch.equal(a, b)
        outs.append(a)
    # the first call's result is reproduced after the scratch held the second call's records
    q, k, v, S_dev = first
    assert torch.equal(_run_noalloc(q, k, v, S_dev, 2), outs[0])


def test_noalloc_rejects_beyond_scratch():
    q = torch.zeros(14, 64, device="cuda")
    big = 1 << 17   # 131072 positions: 2*2048*7*68*4 bytes > 4 MiB
    assert lib.pe_decode_attn_workspace_bytes(14, 2, 64, big) > (4 << 20)
    st = lib.pe_decode_attn_noalloc(_ptr(q), _ptr(q), _ptr(q), 14, 2, 64, big, None, 0, 1,
                                    0.125, 1, _ptr(q), 0, _stream())
    assert st == 6   # PE_ERR_SPACE
