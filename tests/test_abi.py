"""The C ABI (include/pico_hip.h) on a host without a GPU: the library loads, exports every
declared symbol, and rejects bad arguments with the documented status before any launch."""

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = (ROOT / "include" / "pico_hip.h").read_text()


def declared_functions() -> set[str]:
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(pe_\w+)\s*\(", HEADER, re.M))


@pytest.fixture(scope="module")
def lib():
    from pico_hip import _lib
    return _lib.lib


def test_every_declared_symbol_is_exported_and_bound(lib):
    from pico_hip import _lib
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
    assert names == set(_lib.EXPORTED)


def test_status_strings(lib):
    from pico_hip._lib import strerror
    assert strerror(0) == "ok"
    for code in range(1, 7):
        assert strerror(code) and strerror(code) != "unknown pe_status"
    assert strerror(99) == "unknown pe_status"


def test_nbytes_and_workspace(lib):
    assert lib.pe_nbytes_for(12, 4864 * 896) == 2451456
    assert lib.pe_nbytes_for(14, 4864 * 896) == 3575040
    assert lib.pe_nbytes_for(6, 896 * 896) == 551936
    assert lib.pe_nbytes_for(8, 151936 * 896) == 144643072
    assert lib.pe_nbytes_for(12, 896) == -3        # not a whole super-block
    assert lib.pe_nbytes_for(99, 32) == -2         # unknown type
    ws = lib.pe_decode_attn_workspace_bytes(14, 2, 64, 77)
    assert ws == 2 * 2 * 7 * 68 * 4   # records: P.V[64], max, sum, 2 pad words
    assert lib.pe_decode_attn_workspace_bytes(14, 3, 64, 77) == -3   # 14 % 3
    assert lib.pe_decode_attn_workspace_bytes(14, 2, 96, 77) == -3   # head_dim
    assert lib.pe_qgemv_argmax_workspace_bytes(151936) == 256 + 8 * 2048   # grid cap
    assert lib.pe_qgemv_argmax_workspace_bytes(100) == 256 + 8 * 25   # a key per 4-row block
    assert lib.pe_qgemv_argmax_workspace_bytes(0) == -3


def test_argument_errors_before_launch(lib):
    """Invalid calls return a status without touching the GPU (none is present here)."""
    P = ctypes.c_void_p
    fake = P(0x1000)          # never dereferenced: validation fails first
    odd = P(0x1001)
    # unsupported type / bad shapes / NULL / misalignment
    assert lib.pe_qgemv(99, fake, 8, 896, fake, None, None, fake, 0, None) == 2
    assert lib.pe_qgemv(12, fake, 8, 896, fake, None, None, fake, 0, None) == 3   # K % 256
    assert lib.pe_qgemv(8, None, 8, 896, fake, None, None, fake, 0, None) == 1
    assert lib.pe_qgemv(8, odd, 8, 896, fake, None, None, fake, 0, None) == 4
    assert lib.pe_qgemv(8, fake, 8, 896, odd, None, None, fake, 0, None) == 4
    assert lib.pe_qgemv(8, fake, 0, 896, fake, None, None, fake, 0, None) == 3
    assert lib.pe_qgemv(8, fake, 8, 64 * 1024, fake, None, None, fake, 0, None) == 3  # K too large
    assert lib.pe_qgemv(8, fake, 40, 896, fake, None, None, fake, 2, None) == 3  # ut output needs N % 32
    assert lib.pe_qgemv(8, fake, 64, 896, fake, None, None, fake, 4, None) == 2  # unknown layout bit
    assert lib.pe_repack(15, fake, fake, 8, 256, None) == 2                    # Q8_K has no tiled form
    assert lib.pe_dequant(8, fake, fake, 33, None) == 3
    assert lib.pe_dequant(8, fake, fake, 0, None) == 0                         # empty is a no-op
    assert lib.pe_qgemv_rmsnorm(8, fake, 8, 896, fake, None, 1e-6, fake, 0, None) == 1
    assert lib.pe_qgemm(8, fake, 8, 896, fake, 895, 2, None, None, 0, fake, 8, None) == 3  # x_stride < k
    assert lib.pe_embed_gather(8, fake, 10, 896, fake, 0, fake, 0, None) == 0
    assert lib.pe_kv_write(fake, fake, 128, 2, 64, 5, 8, fake, fake, 10, None) == 3  # pos0+L > cap
    assert lib.pe_prefill_attn(fake, 896, fake, fake, 14, 2, 64, 77, 13, 70, 0.125, fake, 896, None) == 3
    ws = lib.pe_decode_attn_workspace_bytes(14, 2, 64, 77)
    assert lib.pe_decode_attn(fake, fake, fake, 14, 2, 64, 77, None, 0, 5, 0.125, 1, fake, fake,
                              ws - 1, 0, None) == 6
    assert lib.pe_decode_attn(fake, fake, fake, 14, 2, 64, 77, None, 3, 5, 0.125, 1, fake, fake,
                              ws, 0, None) == 2
    assert lib.pe_decode_attn(fake, fake, fake, 14, 2, 64, 77, None, 2, 5, 0.125, 1, fake, fake,
                              ws, 0, None) == 1
    assert lib.pe_decode_attn(fake, fake, fake, 14, 2, 64, 77, None, 0, 5, 0.125, 1, fake, fake,
                              ws, 1, None) == 2   # only PE_LAYOUT_Y_UT applies to the output


def test_argmax_argument_errors(lib):
    P = ctypes.c_void_p
    fake = P(0x1000)
    ws = lib.pe_qgemv_argmax_workspace_bytes(4096)
    call = lambda **kw: lib.pe_qgemv_rmsnorm_argmax(
        kw.get("t", 8), fake, kw.get("n", 4096), 896, fake, kw.get("nw", fake), 1e-6, None, fake,
        None, 0, kw.get("ws", fake), kw.get("wsb", ws), kw.get("layout", 0), None)
    assert call(wsb=ws - 1) == 6                  # workspace too small
    assert call(layout=2) == 2                    # the pick needs natural row order
    assert call(nw=None) == 1                     # the LM head always normalises
    assert call(ws=P(0x1010)) == 4                # workspace alignment
    assert call(t=12) == 3                        # Q4_K needs k % 256 == 0
    assert call(n=1 << 31, wsb=1 << 40) == 3      # row ids must fit 31 bits


def test_mqkv_argument_errors(lib):
    """pe_mqkv_rmsnorm_rope and pe_repack_mfma_pairs reject bad calls before any launch."""
    from pico_hip._lib import QkvArgs
    f = 0x1000
    def args(**kw):
        d = dict(type_q=12, type_k=12, type_v=14, w_q=f, w_k=f, w_v=f, b_q=None, b_k=None, b_v=None,
                 x=f, norm_w=f, eps=1e-6, cos_tab=f, sin_tab=f, rope_rows=64, pos=f, q_out=f,
                 k_cache=f, v_cache=f, capacity=40, hidden=3584, n_head=28, n_kv=4, head_dim=128, layout=0)
        d.update(kw)
        return ctypes.byref(QkvArgs(*[d[n] for n, _ in QkvArgs._fields_]))
    call = lambda **kw: lib.pe_mqkv_rmsnorm_rope(args(**kw), None)
    assert call(type_k=14) == 2                 # q and k share a format
    assert call(type_v=6) == 2                  # K-quants only
    assert call(hidden=896) == 3                # whole super-blocks
    assert call(hidden=13824) == 3              # the planes must fit 64 KiB of LDS
    assert call(head_dim=24) == 3               # 16-row groups of whole pairs
    assert call(layout=2) == 3                  # only the input may be unit-transposed
    assert call(norm_w=None) == 1               # the RMSNorm weight is required
    assert call(w_v=None) == 1
    assert call(x=0x1004) == 4                  # 16-byte aligned activation
    assert lib.pe_mqkv_rmsnorm_rope(None, None) == 1
    P = ctypes.c_void_p
    assert lib.pe_repack_mfma_pairs(12, P(f), P(f), 96, 256, 64, None) == 3   # n % head_dim
    assert lib.pe_repack_mfma_pairs(12, P(f), P(f), 96, 256, 24, None) == 3   # head_dim % 16
    assert lib.pe_repack_mfma_pairs(6, P(f), P(f), 64, 256, 64, None) == 3    # no MFMA layout


def test_qkv_embed_argument_errors(lib):
    """pe_qkv_embed_rmsnorm_rope rejects bad embedding and clear arguments before any launch."""
    from pico_hip._lib import QkvArgs
    f = 0x1000
    a = ctypes.byref(QkvArgs(6, 6, 8, f, f, f, None, None, None, None, f, 1e-6, f, f, 64, f, f, f, f, 40,
                             896, 14, 2, 64, 1))
    P = ctypes.c_void_p
    call = lambda et=8, table=f, vocab=100, tok=f, xo=f, clr=f, nb=4096: lib.pe_qkv_embed_rmsnorm_rope(
        a, et, P(table) if table else None, vocab, P(tok) if tok else None, P(xo) if xo else None,
        P(clr) if clr else None, nb, None)
    assert call(et=15) == 2            # Q8_K is not an embedding format here
    assert call(et=12) == 3            # Q4_K rows need hidden % 256 == 0
    assert call(vocab=0) == 3
    assert call(nb=4100) == 3          # whole 16-byte words
    assert call(table=0) == 1
    assert call(tok=0) == 1
    assert call(xo=0) == 1             # the embedding row is stored for the residual
    assert call(clr=0) == 1            # a clear range needs a pointer
    assert call(clr=0x1008) == 4       # 16-byte aligned
    assert call(tok=0x1004) == 4


def test_qkv_args_struct_matches_header():
    """ctypes mirror of pe_qkv_args has the header's fields in the header's order."""
    from pico_hip._lib import QkvArgs
    body = HEADER[HEADER.index("typedef struct pe_qkv_args"):HEADER.index("} pe_qkv_args;")]
    fields = []
    for line in body.splitlines()[1:]:
        decl = line.split("/*")[0].strip().rstrip(";")
        if not decl:
            continue
        names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
        for n in names.split(","):
            fields.append(n.strip().lstrip("*").strip())
    assert [f[0] for f in QkvArgs._fields_] == fields


def test_product_has_no_cpu_fallback():
    """The kernels refuse host tensors instead of computing on the CPU."""
    import torch
    from pico_hip import kernels as K
    with pytest.raises(ValueError, match="GPU tensors"):
        K.rmsnorm(torch.ones(2, 8), torch.ones(8), 1e-6)
    with pytest.raises(ValueError, match="GPU"):
        from pico_hip.model import Transformer
        Transformer(None, {}, torch.device("cpu"), {})


def test_unit_transposed_layout_is_the_documented_permutation():
    import torch
    from pico_hip.kernels import from_ut, to_ut
    n = 896
    v = torch.arange(n, dtype=torch.float32)
    u = to_ut(v)
    U = n // 32
    for k in (0, 1, 3, 4, 31, 32, 100, 895):
        assert u[((k % 32) // 4 * U + k // 32) * 4 + k % 4] == k
    assert torch.equal(from_ut(u), v)
