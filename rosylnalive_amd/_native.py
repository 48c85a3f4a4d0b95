"""ctypes binding of liblrm_hip.so (include/lrm_hip.h), the way the reference's F# side would P/Invoke it.

There is no fallback: when the library is missing this raises, and every compute call goes through the HIP library.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# LRM_HIP_LIB selects another build of the library (the stage-timing variant of rosylnalive_amd/persist_stages.py)
LIB_PATH = os.environ.get("LRM_HIP_LIB") or os.path.join(HERE, "liblrm_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "lrm_hip.h")

LRM_OK, LRM_E_CONTRACT, LRM_E_HIP, LRM_E_ARG, LRM_E_INTERNAL, LRM_E_RANGE = 0, 1, 2, 3, 4, 5
LRM_E_FORMAT, LRM_E_INTEGRITY, LRM_E_DATA = 6, 7, 8


class LrmError(RuntimeError):
    """A failed call into liblrm_hip.so."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class GpuContractException(LrmError):
    """The reference's GpuContractException (src/Lrm.Gpu.Core/Errors.fs:7-13): a broken contract rule."""


class HipDeviceError(LrmError):
    """A device or HIP API failure."""


class SafetensorsFormatError(LrmError):
    """SafetensorsFormatException (src/Lrm.Tensor/Safetensors.fs:15-17): the file breaks a format rule; the message
    names the file and the rule."""


class IntegrityError(LrmError):
    """IntegrityException (Safetensors.fs:20-34): the file's size or SHA-256 differs from the pinned one."""


class TokenizerDataError(LrmError):
    """InvalidDataException of the tokenizer loader (src/Lrm.Tokenizer/TokenizerJson.fs:24-25): tokenizer.json holds
    a configuration this tokenizer does not run."""


class Fp16RangeError(LrmError):
    """A value the fast path stores as fp16 (normed hidden rows, q, the K/V cache, the attention or SwiGLU output)
    became inf or NaN where the float32 reference stays finite: the call's results are not usable. The message names
    the sites."""


class DeviceInfo(C.Structure):
    _fields_ = [
        ("index", C.c_int32),
        ("name", C.c_char * 128),
        ("arch", C.c_char * 64),
        ("vendor_id", C.c_uint32),
        ("pci_device_id", C.c_uint32),
        ("pci_bus", C.c_char * 32),
        ("driver", C.c_char * 64),
        ("memory_bytes", C.c_int64),
        ("compute_units", C.c_int32),
    ]


class QwenConfigC(C.Structure):
    _fields_ = [
        ("layers", C.c_int32),
        ("hidden", C.c_int32),
        ("heads", C.c_int32),
        ("kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("intermediate", C.c_int32),
        ("vocab", C.c_int32),
        ("max_pos", C.c_int32),
        ("eps", C.c_float),
        ("mode", C.c_int32),
        ("max_tokens", C.c_int32),
        ("batch", C.c_int32),
        ("taps", C.c_int32),
    ]


P = C.c_void_p
U32P = C.POINTER(C.c_uint32)
U64P = C.POINTER(C.c_uint64)

# name: (restype, argtypes)
PROTOTYPES = {
    "lrm_last_error": (C.c_char_p, []),
    "lrm_abi_version": (C.c_int, []),
    "lrm_catalog_count": (C.c_int, []),
    "lrm_catalog_find": (C.c_int, [C.c_char_p]),
    "lrm_catalog_kernel": (C.c_int, [C.c_uint32, C.c_char_p, C.c_int, U32P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "lrm_catalog_field": (C.c_int, [C.c_uint32, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int), U32P]),
    "lrm_grid_physical": (C.c_int, [C.c_int, C.c_int64, C.c_int64, C.c_int64, U32P]),
    "lrm_tensor_row": (C.c_int, [C.c_int, C.c_uint64, C.c_uint32, U32P, C.c_int, C.c_uint32, C.c_char_p, U32P]),
    "lrm_debug_id": (C.c_uint32, [C.c_char_p]),
    "lrm_planner_create": (C.c_int, [C.c_uint64, C.POINTER(P)]),
    "lrm_planner_allocate": (C.c_int, [P, C.c_uint32, C.c_uint64, C.POINTER(C.c_int32), U64P]),
    "lrm_planner_build": (C.c_int, [P, U32P, U64P, C.c_int, C.POINTER(C.c_int)]),
    "lrm_planner_destroy": (None, [P]),
    "lrm_table_create": (C.c_int, [U32P, U64P, C.c_int, C.POINTER(P)]),
    "lrm_table_add": (C.c_int, [P, C.c_char_p, C.c_int, C.c_uint64, C.c_uint32, U32P, C.c_int, C.c_uint32, U32P]),
    "lrm_table_add_view": (C.c_int, [P, C.c_char_p, C.c_uint32, U32P, C.c_int, C.c_uint64, U32P]),
    "lrm_table_seal": (C.c_int, [P, P]),
    "lrm_table_destroy": (None, [P]),
    "lrm_prepare": (C.c_int, [P, U32P, U64P, C.c_int, C.c_uint32, U32P, U32P, C.POINTER(C.c_int64), U32P]),
    "lrm_hip_enumerate": (C.c_int, [C.POINTER(DeviceInfo), C.c_int, C.POINTER(C.c_int)]),
    "lrm_hip_create": (C.c_int, [C.c_int, C.c_uint32, C.POINTER(P)]),
    "lrm_hip_destroy": (C.c_int, [P]),
    "lrm_hip_info": (C.c_int, [P, C.POINTER(DeviceInfo)]),
    "lrm_hip_create_heap": (C.c_int, [P, U32P, U64P, C.c_int]),
    "lrm_hip_write_table": (C.c_int, [P, P, C.c_uint64]),
    "lrm_hip_upload": (C.c_int, [P, C.c_int, C.c_uint64, P, C.c_uint64]),
    "lrm_hip_download": (C.c_int, [P, C.c_int, C.c_uint64, P, C.c_uint64]),
    "lrm_hip_load_kernels": (C.c_int, [P, P]),
    "lrm_hip_load_kernel_set": (C.c_int, [P, C.c_uint32, P]),
    "lrm_hip_debug_gemm_stamps": (C.c_int, [P, C.c_uint32, P, C.c_uint64]),
    "lrm_hip_contains": (C.c_int, [P, C.c_uint32]),
    "lrm_hip_denormal_probe": (C.c_int, [P, C.POINTER(C.c_int), U32P]),
    "lrm_hip_begin": (C.c_int, [P, C.c_int, C.POINTER(P)]),
    "lrm_hip_dispatch": (C.c_int, [P, C.c_uint32, U32P]),
    "lrm_hip_dispatch_overlapped": (C.c_int, [P, C.c_uint32, U32P]),
    "lrm_hip_dispatch_decode_attention_static": (C.c_int, [P, U32P, C.c_uint32]),
    "lrm_hip_barrier": (C.c_int, [P]),
    "lrm_hip_copy": (C.c_int, [P, C.c_int, C.c_uint64, C.c_int, C.c_uint64, C.c_uint64]),
    "lrm_hip_begin_timer": (C.c_int, [P, C.c_char_p, C.POINTER(C.c_int)]),
    "lrm_hip_end_timer": (C.c_int, [P, C.c_int]),
    "lrm_hip_submit": (C.c_int, [P, P, C.c_uint32, U64P]),
    "lrm_hip_wait": (C.c_int, [P, C.c_uint64, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "lrm_hip_timer": (C.c_int, [P, C.c_uint64, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "lrm_hip_release": (C.c_int, [P, P]),
    "lrm_qwen_create": (C.c_int, [P, C.POINTER(QwenConfigC), U32P, C.c_int, C.POINTER(P)]),
    "lrm_qwen_destroy": (C.c_int, [P]),
    "lrm_qwen_set_weight": (C.c_int, [P, C.c_char_p, P, C.c_uint64]),
    "lrm_qwen_read_weight": (C.c_int, [P, C.c_char_p, P, C.c_uint64]),
    "lrm_qwen_load_safetensors": (C.c_int, [P, C.c_char_p]),
    "lrm_st_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "lrm_st_open_verified": (C.c_int, [C.c_char_p, C.c_int64, C.c_char_p, C.POINTER(P)]),
    "lrm_st_validate": (C.c_int, [P, C.c_uint64, C.POINTER(P)]),
    "lrm_st_info": (C.c_int, [P, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int32),
                              C.POINTER(C.c_int32), C.POINTER(C.c_int32), U64P]),
    "lrm_st_entry": (C.c_int, [P, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int32), U32P, C.POINTER(C.c_int32),
                               C.POINTER(C.c_int64), C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "lrm_st_metadata": (C.c_int, [P, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int32), C.c_char_p, C.c_int,
                                  C.POINTER(C.c_int32)]),
    "lrm_st_data": (C.c_int, [P, C.c_int, C.POINTER(P)]),
    "lrm_st_close": (C.c_int, [P]),
    "lrm_tok_parse": (C.c_int, [P, C.c_uint64, C.POINTER(P)]),
    "lrm_tok_destroy": (C.c_int, [P]),
    "lrm_tok_info": (C.c_int, [P, C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "lrm_tok_added": (C.c_int, [P, C.c_int, C.POINTER(C.c_int32), C.c_char_p, C.c_int, C.POINTER(C.c_int32),
                                C.POINTER(C.c_int32)]),
    "lrm_tok_encode": (C.c_int, [P, P, C.c_uint64, P, C.c_uint64, U64P]),
    "lrm_tok_encode_bytes": (C.c_int, [P, P, C.c_uint64, P, C.c_uint64, U64P]),
    "lrm_tok_decode_bytes": (C.c_int, [P, P, C.c_uint64, P, C.c_uint64, U64P]),
    "lrm_tok_id_of": (C.c_int, [P, P, C.c_uint64, C.POINTER(C.c_int32)]),
    "lrm_tok_token_of": (C.c_int, [P, C.c_int32, C.c_char_p, C.c_int, C.POINTER(C.c_int32)]),
    "lrm_tok_pre_split": (C.c_int, [P, C.c_uint64, P, C.c_uint64, U64P]),
    "lrm_tok_nfc": (C.c_int, [P, C.c_uint64, P, C.c_uint64, U64P]),
    "lrm_tok_nfc_many": (C.c_int, [P, P, C.c_uint64, P, C.c_uint64, P, U64P]),
    "lrm_tok_scalar_tables": (C.c_int, [P, P, P]),
    "lrm_tok_byte_char": (C.c_int, [C.c_int, U32P]),
    "lrm_qwen_forward": (C.c_int, [P, C.c_int, C.c_int, P, C.c_int, P, C.c_int, U32P]),
    "lrm_qwen_greedy": (C.c_int, [P, P, C.c_int, C.c_int, P]),
    "lrm_qwen_decode_set": (C.c_int, [P, P, P]),
    "lrm_qwen_decode_run": (C.c_int, [P, C.c_int]),
    "lrm_qwen_decode_ids": (C.c_int, [P, P, C.c_int]),
    "lrm_qwen_decode_batch": (C.c_int, [P, P, P, C.c_int, P]),
    "lrm_qwen_read_logits": (C.c_int, [P, P, C.c_int]),
    "lrm_qwen_last_ms": (C.c_double, [P]),
    "lrm_qwen_persistent_decode": (C.c_int, [P]),
    "lrm_qwen_swiglu_shift": (C.c_int, [P]),
    "lrm_qwen_set_swiglu_shift": (C.c_int, [P, C.c_int]),
    "lrm_qwen_token": (C.c_int, [P, C.c_char_p, U32P]),
    "lrm_qwen_device": (P, [P]),
    "lrm_qwen_tap_count": (C.c_int, [P]),
    "lrm_qwen_tap_info": (C.c_int, [P, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int)]),
    "lrm_qwen_read_tap": (C.c_int, [P, C.c_int, P, C.c_int]),
    "lrm_qwen_read_cache": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "lrm_qwen_write_cache": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "lrm_qwen_fill_cache_random": (C.c_int, [P, C.c_uint64, C.c_int]),
    "lrm_stream_of": (C.c_uint64, [C.c_char_p]),
    "lrm_synth_normal_f32": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, P]),
    "lrm_synth_normal_bf16": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, P]),
    "lrm_rope_table": (C.c_int, [U32P, C.c_int, C.c_int, P, P]),
}

_lib = None


def lib():
    """The loaded library. Raises ImportError when liblrm_hip.so has not been built (python -m rosylnalive_amd.build)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m rosylnalive_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == LRM_OK:
        return
    msg = lib().lrm_last_error().decode("utf-8", "replace")
    if rc == LRM_E_CONTRACT:
        raise GpuContractException(rc, msg)
    if rc == LRM_E_HIP:
        raise HipDeviceError(rc, msg)
    if rc == LRM_E_RANGE:
        raise Fp16RangeError(rc, msg)
    if rc == LRM_E_FORMAT:
        raise SafetensorsFormatError(rc, msg)
    if rc == LRM_E_INTEGRITY:
        raise IntegrityError(rc, msg)
    if rc == LRM_E_DATA:
        raise TokenizerDataError(rc, msg)
    if rc == LRM_E_ARG:
        raise LrmError(rc, "invalid argument: " + msg)
    raise LrmError(rc, msg)


def u32s(values) -> "C.Array":
    vals = list(values)
    return (C.c_uint32 * max(1, len(vals)))(*vals)


def u64s(values) -> "C.Array":
    vals = list(values)
    return (C.c_uint64 * max(1, len(vals)))(*vals)
