"""ctypes binding of ``libfaquant_amd.so`` (the C ABI in include/faquant_amd.h).

The library is built in-tree by ``faquant-public_amd/build.py``.  There is no
fallback: if the library is missing or a tensor is not on a ROCm device, the
call raises.  Status codes map to the exception types the reference raises
for the same conditions (ValueError / NotImplementedError).
"""

from __future__ import annotations

import ctypes
import os

import torch

LIB_NAME = "libfaquant_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

F32, BF16, F16 = 0, 1, 2
_DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

OK, EINVAL, EUNSUP, ELAUNCH = 0, -1, -2, -3

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_vp = ctypes.c_void_p



class AttnOpts(ctypes.Structure):
    """``faq_attn_opts``: key-range masks and the logit softcap of the attention kernel."""

    _fields_ = [
        ("row_lo", _vp),
        ("row_hi", _vp),
        ("row_blocks", _vp),
        ("key_bits", _vp),
        ("key_words", _c_i64),
        ("softcap", _c_float),
        ("pv_probe", _vp),
        ("dense_mask", _vp),
        ("dm_sb", _c_i64),
        ("dm_sh", _c_i64),
        ("dm_sq", _c_i64),
        ("p_dump", _vp),
        ("p_dump_stride", _c_i64),
        ("q_prep", _c_int),
        ("q_hadamard", _c_int),
        ("q_levels", _c_int),
    ]


_opts_p = ctypes.POINTER(AttnOpts)


class HiF4KV(ctypes.Structure):
    """``faq_hif4_kv``: a packed HiF4 K or V cache (code and meta words, row strides)."""

    _fields_ = [("codes", _vp), ("meta", _vp), ("sb", _c_i64), ("sh", _c_i64)]


_kv_p = ctypes.POINTER(HiF4KV)


class ActOpts(ctypes.Structure):
    """``faq_act_opts``: the optional steps of the full Linear activation path."""

    _fields_ = [
        ("col_scale", _vp),
        ("rot_signs", _vp),
        ("rot_perm", _vp),
        ("rot_block", _c_int),
        ("has_min", _c_int),
        ("has_max", _c_int),
        ("act_min", _c_float),
        ("act_max", _c_float),
        ("compand", _vp),
        ("hadamard", _c_int),
        ("hadamard_generalized", _c_int),
        ("compand_rcp", _vp),
        ("stage_round", _c_int),
    ]


_act_opts_p = ctypes.POINTER(ActOpts)

_SIGNATURES = {
    "faq_last_error": ([], ctypes.c_char_p),
    "faq_version": ([], ctypes.c_char_p),
    "faq_hif4_qdq_rows": (
        [_vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
        _c_int,
    ),
    "faq_hadamard_rows": ([_vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _vp], _c_int),
    "faq_hadamard_rows_native": ([_vp, _vp, _c_i64, _c_i64, _c_int, _vp], _c_int),
    "faq_act_qdq_rows": ([_vp, _vp, _c_i64, _c_i64, _c_int, _vp, _c_int, _c_int, _vp], _c_int),
    "faq_act_prep_rows": ([_vp, _vp, _c_i64, _c_i64, _c_int, _act_opts_p, _c_int, _vp], _c_int),
    "faq_act_compand_rcp": ([_vp, _vp, _c_i64, _c_int, _vp], _c_int),
    "faq_hif4_unpack_rows": ([_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_int, _vp, _vp], _c_int),
    "faq_operand_prep": (
        [
            _vp, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int,
            _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_int, _vp,
        ],
        _c_int,
    ),
    "faq_operand_prep_vt": (
        [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_int, _vp],
        _c_int,
    ),
    "faq_operand_prep_hif4_kv": (
        [
            _vp, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int,
            _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_i64, _c_i64, _vp,
        ],
        _c_int,
    ),
    "faq_attention_decode_workspace": ([_c_int, _c_int, _c_int, _c_int, _c_int], _c_i64),
    "faq_attention_decode": (
        [
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64,
            _kv_p, _kv_p,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_int, _vp,
            _c_int, _vp, _c_i64, _vp,
        ],
        _c_int,
    ),
    "faq_hif4_linear_packed": (
        [_vp, _c_i64, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _vp],
        _c_int,
    ),
    "faq_attention_split_workspace": ([_c_int, _c_int, _c_int, _c_int, _c_int], _c_i64),
    "faq_mfma_probe": ([_vp, _c_int, _c_int, _vp], _c_int),
    "faq_stream_probe": ([_vp, _c_i64, _vp, _c_int, _vp], _c_int),
    "faq_pquant_groups": ([_vp, _vp, _c_i64, _c_int, _vp], _c_int),
    "faq_attention_fwd_split": (
        [
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64, _c_int,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_int, _vp,
            _c_int, _vp, _c_i64, _opts_p, _vp,
        ],
        _c_int,
    ),
    "faq_attention_fwd_split_noalloc": (
        [
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64, _c_int,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_int, _vp,
            _c_int, _opts_p, _vp,
        ],
        _c_int,
    ),
    "faq_attention_mask_bounds": (
        [_vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_i64, _vp],
        _c_int,
    ),
    "faq_attention_fwd_general": (
        [
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_int, _vp,
            _opts_p, _vp,
        ],
        _c_int,
    ),
    "faq_attention_fwd": (
        [
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64,
            _vp, _c_i64, _c_i64, _c_i64, _c_int,
            _vp, _c_int, _c_i64, _c_i64, _c_i64,
            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_int, _vp, _c_int,
            _opts_p, _vp,
        ],
        _c_int,
    ),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python faquant-public_amd/build.py, or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status == OK:
        return
    message = load().faq_last_error().decode(errors="replace")
    if status == EUNSUP:
        raise NotImplementedError(message)
    if status == EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(
                "faquant_amd kernels run on the MI355X: move tensors to a ROCm device "
                "(this build has no CPU path)"
            )


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _ForwardOnly(torch.autograd.Function):
    """A result of the forward-only HIP path, joined to the autograd graph of its inputs: a
    backward pass through it raises instead of silently giving those inputs no gradient
    (the reference's simulator is differentiable; this build implements inference)."""

    @staticmethod
    def forward(ctx, result, *inputs):
        return result.view_as(result)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("the HIP HiF4 path is forward-only: backward is not implemented")


def forward_only(result: torch.Tensor, *inputs) -> torch.Tensor:
    """`result`, tracked by autograd when grad mode is on and an input requires grad."""
    tracked = [t for t in inputs if isinstance(t, torch.Tensor) and t.requires_grad]
    if torch.is_grad_enabled() and tracked:
        return _ForwardOnly.apply(result, *tracked)
    return result


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
