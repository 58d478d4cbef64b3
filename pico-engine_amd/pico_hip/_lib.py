"""ctypes binding of libpico_hip.so (the C ABI declared in include/pico_hip.h).

torch is imported first on purpose: torch ships the HIP runtime (libamdhip64.so.7), and
loading it before this library makes the dynamic linker resolve our dependency to that same
runtime, so the streams and device pointers torch hands us are valid here. There is no
fallback: if the library is missing, importing this module raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpico_hip.so")

# layout bits (include/pico_hip.h)
LAYOUT_NATURAL, LAYOUT_X_UT, LAYOUT_Y_UT = 0, 1, 2
ABI_VERSION = 3

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float


class PicoHipError(RuntimeError):
    """A libpico_hip entry point returned a non-zero pe_status."""

    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} (pe_status {status})")


class QkvArgs(ctypes.Structure):
    """Mirror of pe_qkv_args (include/pico_hip.h)."""

    _fields_ = [
        ("type_q", _I), ("type_k", _I), ("type_v", _I),
        ("w_q", _P), ("w_k", _P), ("w_v", _P),
        ("b_q", _P), ("b_k", _P), ("b_v", _P),
        ("x", _P), ("norm_w", _P), ("eps", _F),
        ("cos_tab", _P), ("sin_tab", _P), ("rope_rows", _L),
        ("pos", _P), ("q_out", _P), ("k_cache", _P), ("v_cache", _P),
        ("capacity", _L), ("hidden", _L),
        ("n_head", _I), ("n_kv", _I), ("head_dim", _I),
        ("layout", _I),
    ]


class AttnOprojArgs(ctypes.Structure):
    """Mirror of pe_attn_oproj_args (include/pico_hip.h)."""

    _fields_ = [
        ("q", _P), ("k_cache", _P), ("v_cache", _P), ("capacity", _L), ("pos", _P),
        ("n_head", _I), ("n_kv", _I), ("head_dim", _I), ("scale", _F),
        ("type_o", _I), ("w_o", _P), ("hidden", _L), ("acc", _P), ("layout", _I),
    ]


class StepLayer(ctypes.Structure):
    """Mirror of pe_step_layer (include/pico_hip.h)."""

    _fields_ = [
        ("type_q", _I), ("type_k", _I), ("type_v", _I), ("type_o", _I), ("type_gu", _I),
        ("type_down", _I),
        ("w_q", _P), ("w_k", _P), ("w_v", _P), ("w_o", _P), ("w_gu", _P), ("w_down", _P),
        ("b_q", _P), ("b_k", _P), ("b_v", _P),
        ("attn_norm", _P), ("ffn_norm", _P),
        ("k_cache", _P), ("v_cache", _P),
    ]


class StepArgs(ctypes.Structure):
    """Mirror of pe_step_args (include/pico_hip.h)."""

    _fields_ = [
        ("layers", ctypes.POINTER(StepLayer)), ("layers_dev", _P),
        ("n_layers", _I), ("hidden", _I), ("ffn", _I), ("n_head", _I), ("n_kv", _I),
        ("head_dim", _I),
        ("capacity", _L), ("vocab", _L), ("rope_rows", _L),
        ("eps", _F), ("scale", _F),
        ("embed_type", _I), ("embed", _P),
        ("out_type", _I), ("w_out", _P), ("out_norm", _P),
        ("cos_tab", _P), ("sin_tab", _P),
        ("state", _P), ("log", _P), ("log_cap", _L),
        ("logits", _P),
        ("workspace", _P), ("workspace_bytes", _L),
        ("n_wg", _I),
    ]


class FfnFixArgs(ctypes.Structure):
    """Mirror of pe_ffn_fix_args (include/pico_hip.h)."""

    _fields_ = [
        ("type_gu", _I), ("w_gu", _P), ("type_down", _I), ("w_down", _P),
        ("hidden", _L), ("ffn", _L),
        ("x", _P), ("acc_in", _P), ("norm_w", _P), ("eps", _F), ("x_sum", _P),
        ("acc_out", _P), ("replicas", _I), ("acc_stride", _L), ("layout", _I),
    ]


_SIGNATURES = {
    "pe_strerror": (ctypes.c_char_p, [_I]),
    "pe_abi_version": (_I, []),
    "pe_nbytes_for": (_L, [_I, _L]),
    "pe_dequant": (_I, [_I, _P, _P, _L, _P]),
    "pe_repack": (_I, [_I, _P, _P, _L, _L, _P]),
    "pe_dequant_tiled": (_I, [_I, _P, _P, _L, _L, _P]),
    "pe_dequant_tiled_f16": (_I, [_I, _P, _P, _L, _L, _P]),
    "pe_gemm_f16": (_I, [_P, _L, _P, _P, _P, _L, _P, _L, _L, _L, _L, _P]),
    "pe_gemm_f16_silu": (_I, [_P, _L, _P, _P, _L, _L, _L, _L, _P]),
    "pe_gemm_f16_silu_h": (_I, [_P, _L, _P, _P, _L, _L, _L, _L, _P]),
    "pe_gemm_h16_silu_h": (_I, [_P, _L, _P, _P, _L, _L, _L, _L, _P]),
    "pe_gemm_h16": (_I, [_P, _L, _P, _P, _P, _L, _P, _L, _L, _L, _L, _P]),
    "pe_flash_prefill": (_I, [_P, _L, _P, _P, _I, _I, _I, _L, _L, _L, _F, _P, _L, _P]),
    "pe_flash_prefill_h16": (_I, [_P, _L, _P, _P, _I, _I, _I, _L, _L, _L, _F, _P, _L, _P]),
    "pe_flash_prefill_blocks": (_I, [_P, _L, _P, _L, _I, _I, _I, _L, _F, _P, _L, _P, _L, _P]),
    "pe_flash_prefill_blocks_workspace": (_L, [_I, _I, _L]),
    "pe_gemm_lt": (_I, [_P, _L, _P, _L, _L, _L, _P, _P, _L, _P, _L, _P, _L, _P]),
    "pe_gemm_lt_init": (_I, []),
    "pe_mfma_bytes": (_L, [_I, _L, _L]),
    "pe_repack_mfma": (_I, [_I, _P, _P, _L, _L, _P]),
    "pe_repack_mfma_pairs": (_I, [_I, _P, _P, _L, _L, _I, _P]),
    "pe_mgemv": (_I, [_I, _P, _L, _L, _P, _P, _F, _P, _P, _I, _I, _P]),
    "pe_embed_gather": (_I, [_I, _P, _L, _L, _P, _L, _P, _I, _P]),
    "pe_qgemv": (_I, [_I, _P, _L, _L, _P, _P, _P, _P, _I, _P]),
    "pe_qgemv_rmsnorm": (_I, [_I, _P, _L, _L, _P, _P, _F, _P, _I, _P]),
    "pe_qgemv_rmsnorm_silu": (_I, [_I, _P, _L, _L, _P, _P, _F, _P, _I, _P]),
    "pe_qgemv_argmax_workspace_bytes": (_L, [_L]),
    "pe_qgemv_rmsnorm_argmax": (_I, [_I, _P, _L, _L, _P, _P, _F, _P, _P, _P, _L, _P, _L, _I, _P]),
    "pe_qkv_rmsnorm_rope": (_I, [ctypes.POINTER(QkvArgs), _P]),
    "pe_mqkv_rmsnorm_rope": (_I, [ctypes.POINTER(QkvArgs), _P]),
    "pe_decode_attn_workspace_bytes": (_L, [_I, _I, _I, _L]),
    "pe_decode_attn": (_I, [_P, _P, _P, _I, _I, _I, _L, _P, _I, _L, _F, _I, _P, _P, _L, _I, _P]),
    "pe_decode_attn_noalloc": (_I, [_P, _P, _P, _I, _I, _I, _L, _P, _I, _L, _F, _I, _P, _I, _P]),
    "pe_qgemv_sum_rmsnorm_silu": (_I, [_I, _P, _L, _L, _P, _P, _I, _P, _F, _P, _P, _I, _P]),
    "pe_attn_gproj_supported": (_I, [_I, _I, _I, _L, _I, _L]),
    "pe_attn_gproj": (_I, [_P, _P, _P, _I, _I, _I, _L, _P, _I, _L, _F, _I, _I, _P, _L, _P, _I, _P]),
    "pe_attn_split_gproj_supported": (_I, [_I, _I, _I, _L, _I, _L]),
    "pe_attn_split_gproj": (_I, [_P, _P, _P, _I, _I, _I, _L, _P, _I, _L, _F, _I, _I, _P, _L, _P, _P, _L, _I, _P]),
    "pe_rmsnorm": (_I, [_P, _L, _P, _P, _L, _L, _L, _F, _P]),
    "pe_rmsnorm_h16": (_I, [_P, _L, _P, _P, _L, _L, _L, _F, _P]),
    "pe_rope": (_I, [_P, _L, _P, _P, _P, _L, _L, _I, _I, _P]),
    "pe_silu_mul": (_I, [_P, _L, _P, _L, _L, _L, _P]),
    "pe_round_f16": (_I, [_P, _L, _L, _L, _P]),
    "pe_qgemm": (_I, [_I, _P, _L, _L, _P, _L, _L, _P, _P, _L, _P, _L, _P]),
    "pe_kv_write": (_I, [_P, _P, _L, _I, _I, _L, _L, _P, _P, _L, _P]),
    "pe_rope_kv_write": (_I, [_P, _L, _P, _P, _I, _I, _I, _L, _L, _P, _P, _P, _L, _P]),
    "pe_rope_kv_write_blocks": (_I, [_P, _L, _P, _P, _I, _I, _I, _L, _L, _P, _P, _P, _L, _P, _L, _P]),
    "pe_prefill_attn": (_I, [_P, _L, _P, _P, _I, _I, _I, _L, _L, _L, _F, _P, _L, _P]),
    "pe_decode_step_supported": (_I, [_I, _I, _I, _I, _I, _I, _L, _L]),
    "pe_decode_step_workspace_bytes": (_L, [_I, _I, _I, _I, _I, _I]),
    "pe_decode_step": (_I, [ctypes.POINTER(StepArgs), _P]),
    "pe_oproj_layout_bytes": (_L, [_I, _L, _L]),
    "pe_repack_oproj": (_I, [_I, _P, _P, _L, _L, _P]),
    "pe_attn_oproj_fix_supported": (_I, [_I, _L, _I, _I, _I, _L]),
    "pe_attn_oproj_fix": (_I, [ctypes.POINTER(AttnOprojArgs), _P]),
    "pe_qgemv_fix_rmsnorm_silu": (_I, [_I, _P, _L, _L, _P, _P, _P, _F, _P, _P, _I, _P]),
    "pe_down_slice_bytes": (_L, [_I, _L, _L]),
    "pe_repack_down_slices": (_I, [_I, _P, _P, _L, _L, _P]),
    "pe_ffn_fix_supported": (_I, [_I, _I, _L, _L]),
    "pe_ffn_fix_bound": (_F, [_L]),
    "pe_ffn_fix": (_I, [ctypes.POINTER(FfnFixArgs), _P]),
    "pe_qkv_fix_rmsnorm_rope": (_I, [ctypes.POINTER(QkvArgs), _P, _I, _L, _P, _P]),
    "pe_qkv_embed_rmsnorm_rope": (_I, [ctypes.POINTER(QkvArgs), _I, _P, _L, _P, _P, _P, _L, _P]),
}

# Every symbol include/pico_hip.h declares (checked by tests/test_abi.py).
EXPORTED = tuple(_SIGNATURES)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; build it with `make -C pico-engine_amd -j8` "
            "or __graft_entry__.build() (there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.pe_abi_version() != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {lib.pe_abi_version()} != {ABI_VERSION}")
    return lib


lib = _load()


def strerror(status: int) -> str:
    return lib.pe_strerror(int(status)).decode()


def check(status: int, what: str) -> None:
    if status != 0:
        raise PicoHipError(int(status), what)
