"""ctypes binding of libqwen_state.so (the C ABI declared in include/qwen_state.h).

The library is the only compute path: if it is missing or fails to load, every op raises. There is no
CPU or PyTorch fallback.
"""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqwen_state.so")

_P, _I, _F, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes), in the order of include/qwen_state.h
SIGNATURES = {
    "qs_abi_version": (_I, []),
    "qs_last_error": (ctypes.c_char_p, []),
    "qs_conv1d_update": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "qs_gdn_gates": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "qs_gdn_decode_step": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P]),
    "qs_gdn_workspace_bytes": (_Z, [_I, _I]),
    "qs_gdn_decode_fused": (
        _I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _P]),
    "qs_gdn_decode_fused_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _P]),
    "qs_gdn_noalloc_scratch_read": (_I, [_P, _I, _P]),
    "qs_gdn_gated_norm": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "qs_gdn_verify_step": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _F, _P],
    ),
    "qs_gdn_verify_step_slots": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _F, _P],
    ),
    "qs_verify_accept": (_I, [_P, _P, _P, _P, _I, _I, _P, _P]),
    "qs_gdn_rollback": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "qs_gdn_rollback_layers": (
        _I, [_P, _Z, _P, _Z, _P, _Z, _P, _Z, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "qs_paged_kv_append": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "qs_advance_lengths": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "qs_paged_kv_fill": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "qs_paged_kv_gather": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "qs_paged_attention_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I, _I]),
    "qs_paged_gqa_decode": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P],
    ),
    "qs_attn_mixer_decode": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P],
    ),
    "qs_gdn_chunk_prefill_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I]),
    "qs_gdn_chunk_prefill": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _P],
    ),
    "qs_conv1d_prefill": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "qs_mx_packed_bytes": (_Z, [_I, _I, _I]),
    "qs_mx_quantize": (_I, [_P, _P, _I, _I, _I, _P]),
    "qs_mx_gemv_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "qs_mx_gemv": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "qs_mlp_decode_workspace_bytes": (_Z, [_I, _I, _I]),
    "qs_mlp_decode": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _F, _P]),
    "qs_probe_sink_words": (_Z, [_Z]),
    "qs_probe_read": (_I, [_P, _Z, _P, _P]),
    "qs_probe_copy": (_I, [_P, _P, _Z, _P]),
    "qs_probe_gather_sink_words": (_Z, [_I, _I, _I, _I]),
    "qs_probe_gather": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P]),
}

_lib = None


class QSError(RuntimeError):
    """A call into libqwen_state returned a non-zero status."""


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python tt-qwen-resident_amd/qwen36_state/build.py` "
                "(or __graft_entry__.build()) — there is no fallback path"
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def call(name, *args):
    """Call ``name``; raise ValueError (invalid argument) or QSError (HIP error) on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().qs_last_error().decode()
        if rc == -1:
            raise ValueError(msg)
        raise QSError(f"{name} failed ({rc}): {msg}")
    return rc
