"""ctypes binding of libpcp_grpo.so (the C ABI declared in include/pcp_grpo.h).

The library is built in-tree (``make -C pcp_amd/csrc`` or ``__graft_entry__.build()``)
and loaded from this package directory. There is no fallback: if the library is
missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import enum
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# PCP_GRPO_LIB selects another build of the same library (the host-sanitizer build of
# the CPU test run); by default the in-tree one.
LIB_PATH = os.environ.get("PCP_GRPO_LIB") or os.path.join(_HERE, "libpcp_grpo.so")


class DType(enum.IntEnum):
    """Element types in the order of DType, src/core/tensor.zig:9-16."""
    f16 = 0
    bf16 = 1
    f32 = 2
    f64 = 3
    i32 = 4
    i64 = 5
    bool = 6

    def size_in_bytes(self) -> int:  # tensor.zig:50-60
        return {0: 2, 1: 2, 2: 4, 3: 8, 4: 4, 5: 8, 6: 1}[int(self)]


class Backend(enum.IntEnum):
    """Backend kinds in the order of Backend, src/backends/selection.zig:32-38."""
    metal = 0
    cuda = 1
    vulkan = 2
    rocm = 3
    cpu = 4


class LossMode(enum.IntEnum):
    REINFORCE = 0
    GRPO_CLIP_KL = 1


FLAG_ASYNC = 0x1
FLAG_NO_ZERO_FILL = 0x2
FLAG_FORCE_STREAMING = 0x4
FLAG_EXACT_BF16 = 0x8
NOALLOC_SCRATCH_BYTES = 4 << 20
IGNORE_INDEX = -100

STATUS = {
    0: "PCP_OK",
    -1: "PCP_ERR_INVALID_ARG",
    -2: "PCP_ERR_DTYPE",
    -3: "PCP_ERR_TOKEN_RANGE",
    -4: "PCP_ERR_NONFINITE",
    -5: "PCP_ERR_OOM",
    -6: "PCP_ERR_DEVICE",
    -7: "PCP_ERR_UNKNOWN_FUNCTION",
    -8: "PCP_ERR_COUNT_MISMATCH",
    -9: "PCP_ERR_OVERFLOW",
    -10: "PCP_ERR_UNSUPPORTED",
    -11: "PCP_ERR_OUT_OF_BOUNDS",
    -12: "PCP_ERR_DIMENSION_MISMATCH",
    -13: "PCP_ERR_CORRUPT_STATE",
    -14: "PCP_ERR_IO",
}


class PcpError(RuntimeError):
    """A negative pcp_status; ``code`` and ``name`` identify it."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.name = STATUS.get(code, f"status {code}")
        super().__init__(f"{self.name}: {message}")


class GrpoArgs(ctypes.Structure):
    """pcp_grpo_args (field order and types as in include/pcp_grpo.h)."""
    _fields_ = [
        ("n_seq", ctypes.c_int64), ("rows", ctypes.c_int64), ("vocab", ctypes.c_int64),
        ("group_size", ctypes.c_int64), ("logit_seq_stride", ctypes.c_int64),
        ("tok_seq_stride", ctypes.c_int64), ("tok_offset", ctypes.c_int64),
        ("logits_dtype", ctypes.c_int32), ("dlogits_dtype", ctypes.c_int32),
        ("ids_dtype", ctypes.c_int32), ("mask_dtype", ctypes.c_int32),
        ("logits", ctypes.c_void_p), ("ref_logits", ctypes.c_void_p), ("ids", ctypes.c_void_p),
        ("mask", ctypes.c_void_p), ("old_logp", ctypes.c_void_p), ("advantages", ctypes.c_void_p),
        ("rewards", ctypes.c_void_p),
        ("dlogits", ctypes.c_void_p), ("logp", ctypes.c_void_p), ("ref_logp", ctypes.c_void_p),
        ("token_loss", ctypes.c_void_p), ("advantages_out", ctypes.c_void_p), ("loss", ctypes.c_void_p),
        ("loss_mode", ctypes.c_int32), ("clip_eps", ctypes.c_float), ("kl_beta", ctypes.c_float),
        ("std_eps", ctypes.c_float), ("loss_norm", ctypes.c_float), ("flags", ctypes.c_uint32),
        ("stream", ctypes.c_void_p),
    ]


class LmheadArgs(ctypes.Structure):
    """pcp_lmhead_args (field order and types as in include/pcp_grpo.h)."""
    _fields_ = [
        ("n_seq", ctypes.c_int64), ("rows", ctypes.c_int64), ("hidden", ctypes.c_int64),
        ("vocab", ctypes.c_int64), ("group_size", ctypes.c_int64), ("vocab_chunk", ctypes.c_int64),
        ("ids_dtype", ctypes.c_int32), ("mask_dtype", ctypes.c_int32),
        ("hidden_states", ctypes.c_void_p), ("weight", ctypes.c_void_p), ("ref_weight", ctypes.c_void_p),
        ("ids", ctypes.c_void_p), ("mask", ctypes.c_void_p), ("old_logp", ctypes.c_void_p),
        ("advantages", ctypes.c_void_p), ("rewards", ctypes.c_void_p),
        ("logp", ctypes.c_void_p), ("ref_logp", ctypes.c_void_p), ("token_loss", ctypes.c_void_p),
        ("advantages_out", ctypes.c_void_p), ("loss", ctypes.c_void_p),
        ("dhidden", ctypes.c_void_p), ("dweight", ctypes.c_void_p),
        ("loss_mode", ctypes.c_int32), ("clip_eps", ctypes.c_float), ("kl_beta", ctypes.c_float),
        ("std_eps", ctypes.c_float), ("loss_norm", ctypes.c_float), ("flags", ctypes.c_uint32),
        ("stream", ctypes.c_void_p),
        ("norm_weight", ctypes.c_void_p), ("dnorm_weight", ctypes.c_void_p), ("norm_eps", ctypes.c_float),
    ]


class GradStats(ctypes.Structure):
    """pcp_grad_stats (include/pcp_step.h)."""
    _fields_ = [
        ("sumsq", ctypes.c_double), ("l2_norm", ctypes.c_double), ("max_abs", ctypes.c_float),
        ("nan_count", ctypes.c_int64), ("inf_count", ctypes.c_int64), ("elements", ctypes.c_int64),
    ]


class NesterovMode(enum.IntEnum):
    sutskever = 0   # nesterov.zig:86-97 (RLShepherd's optimizer)
    mlir = 1        # nesterov_mlir.zig:93-99


# Every symbol the headers in include/ declare, with its ctypes signature.
_VP, _I, _I64, _F, _U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_uint64
SIGNATURES = {
    "pcp_grpo_args_init": (None, [ctypes.POINTER(GrpoArgs)]),
    "pcp_init": (_I, [_I, _I, ctypes.POINTER(_VP)]),
    "pcp_destroy": (None, [_VP]),
    "pcp_get_backend_type": (_I, [_VP]),
    "pcp_last_error": (ctypes.c_char_p, [_VP]),
    "pcp_sync": (_I, [_VP]),
    "pcp_release_workspace": (_I, [_VP]),
    "pcp_workspace_bytes": (ctypes.c_size_t, [_VP]),
    "pcp_execute": (_I, [_VP, ctypes.c_char_p, _I, ctypes.POINTER(_VP), ctypes.POINTER(ctypes.c_size_t),
                         ctypes.POINTER(ctypes.POINTER(_I64)), ctypes.POINTER(_I), ctypes.POINTER(_I),
                         ctypes.POINTER(_I), ctypes.POINTER(ctypes.POINTER(_VP)),
                         ctypes.POINTER(ctypes.POINTER(ctypes.c_size_t))]),
    "pcp_free": (None, [_VP, _I, ctypes.POINTER(_VP), ctypes.POINTER(ctypes.c_size_t)]),
    "pcp_grpo_logprob_fwd": (_I, [_VP, ctypes.POINTER(GrpoArgs)]),
    "pcp_grpo_advantages": (_I, [_VP, _VP, _I64, _I64, _F, _VP, _VP]),
    "pcp_grpo_loss_fwd_bwd": (_I, [_VP, ctypes.POINTER(GrpoArgs)]),
    "pcp_grpo_loss_fwd_bwd_noalloc": (_I, [_VP, ctypes.POINTER(GrpoArgs)]),
    "pcp_lmhead_args_init": (None, [ctypes.POINTER(LmheadArgs)]),
    "pcp_grpo_lmhead_fwd_bwd": (_I, [_VP, ctypes.POINTER(LmheadArgs)]),
    "pcp_profile_start": (_I, [_VP, _I]),
    "pcp_profile_stop": (_I, [_VP, ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_double)]),
    "pcp_version": (ctypes.c_char_p, []),
    "pcp_synth_philox4x32_10": (None, [ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                       ctypes.POINTER(ctypes.c_uint32)]),
    "pcp_synth_logits": (_I, [_VP, _VP, _I64, _I, _F, _F, _U64, _VP]),
    "pcp_synth_sample_tokens": (_I, [_VP, _I, _I64, _I64, _U64, _VP, _VP]),
    "pcp_synth_lmhead_tokens": (_I, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _U64, _VP, _VP]),
    "pcp_hbm_stream": (_I, [_VP, _I, _I, _I, _VP, _VP, _VP, _I64, _VP]),
    "pcp_mfma_peak": (_I, [_VP, _I, _I, _I, ctypes.c_uint32, _VP, _VP, _VP]),
    "pcp_pack_rollouts": (_I, [_VP, _VP, _I64, _VP, _VP, _I64, _VP, _I64, _I64, _I64, _VP, _VP, _VP]),
    "pcp_grad_stats_compute": (_I, [_VP, _VP, _I64, _I, ctypes.POINTER(GradStats), _VP]),
    "pcp_nesterov_create": (_I, [_VP, _F, _F, _I, _I, ctypes.POINTER(_I64), ctypes.POINTER(_VP)]),
    "pcp_nesterov_destroy": (None, [_VP]),
    "pcp_nesterov_reset": (_I, [_VP, _VP]),
    "pcp_nesterov_update": (_I, [_VP, _I, _VP, _VP, _I64, _VP]),
    "pcp_nesterov_update_flat": (_I, [_VP, _VP, _VP, _VP, _VP]),
    "pcp_nesterov_total": (_I64, [_VP]),
    "pcp_nesterov_serialize": (_I, [_VP, _VP, ctypes.c_size_t]),
    "pcp_nesterov_deserialize": (_I, [_VP, _VP, ctypes.c_size_t]),
    "pcp_sample_tokens": (_I, [_VP, _VP, _I, _I64, _I64, _I64, _F, _VP, _VP, _VP]),
    "pcp_sample_tokens_async": (_I, [_VP, _VP, _I, _I64, _I64, _I64, _F, _VP, _VP, _VP]),
    "pcp_prompts_load": (_I, [_VP, ctypes.c_char_p, _VP, _I64, _VP, _I64, ctypes.POINTER(_I64),
                              ctypes.POINTER(_I64)]),
    "pcp_weights_load": (_I, [_VP, ctypes.c_char_p, _I, ctypes.POINTER(_I64), _VP, _VP]),
    "pcp_weights_save": (_I, [_VP, ctypes.c_char_p, _VP, _I64]),
    "pcp_base64_encoded_len": (_I64, [_I64]),
    "pcp_base64_encode": (_I, [_VP, _VP, _I64, _VP, _VP]),
    "pcp_base64_decode": (_I, [_VP, _VP, _I64, _VP, ctypes.POINTER(_I64), _VP]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libpcp_grpo.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP library first (make -C pcp_amd/csrc, "
                "or __graft_entry__.build()). There is no non-HIP fallback.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, ctx=None) -> None:
    """Raise PcpError for a negative status, with the library's message."""
    if rc != 0:
        msg = lib().pcp_last_error(ctx)
        raise PcpError(rc, msg.decode() if msg else "")


def default_args() -> GrpoArgs:
    a = GrpoArgs()
    lib().pcp_grpo_args_init(ctypes.byref(a))
    return a
