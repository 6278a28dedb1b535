"""ctypes binding of ``libgemmkit_hip.so`` (declared in ``include/gemmkit_hip.h``).

Loading the library needs no GPU; calling a compute entry point does.  There is
no fallback: when the library is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# GEMMKIT_HIP_LIBRARY names another build of the same ABI (A/B comparisons).
LIB_PATH = os.environ.get("GEMMKIT_HIP_LIBRARY") or os.path.join(_HERE, "libgemmkit_hip.so")

_size = C.c_size_t
_sdiff = C.c_ssize_t
_vp = C.c_void_p
_i32 = C.c_int32
_u32 = C.c_uint32
_u16 = C.c_uint16
_f32 = C.c_float
_u8 = C.c_uint8


class MatRefC(C.Structure):
    """``gk_mat_ref``: MatRef (src/api.rs:92-180) with its slice length."""
    _fields_ = [("data", _vp), ("len", _size), ("rows", _size), ("cols", _size),
                ("rs", _sdiff), ("cs", _sdiff)]


class MatMutC(C.Structure):
    """``gk_mat_mut``: MatMut (src/api.rs:92-180) with its slice length."""
    _fields_ = [("data", _vp), ("len", _size), ("rows", _size), ("cols", _size),
                ("rs", _sdiff), ("cs", _sdiff)]


class RequantizeC(C.Structure):
    """``gk_requantize``: Requantize (src/api/int8.rs:185-209) plus axis/act."""
    _fields_ = [("scale", _f32), ("scales", _vp), ("scales_len", _size),
                ("zero_point", _i32), ("bias", _vp), ("bias_len", _size),
                ("axis", _i32), ("act", _i32)]


class BiasC(C.Structure):
    """``gk_bias``: Bias::PerRow / PerCol (src/api/fused.rs:17-23) with its length."""
    _fields_ = [("data", _vp), ("len", _size), ("dim", _i32)]


class ProblemF32C(C.Structure):
    """``gk_problem_f32``: GemmProblem<f32> (src/dispatch.rs:135-164)."""
    _fields_ = [("m", _size), ("k", _size), ("n", _size), ("alpha", _f32), ("a", _vp),
                ("rsa", _sdiff), ("csa", _sdiff), ("b", _vp), ("rsb", _sdiff), ("csb", _sdiff),
                ("beta", _f32), ("c", _vp), ("rsc", _sdiff), ("csc", _sdiff)]


class ProblemBf16C(C.Structure):
    """``gk_problem_bf16``: GemmProblem<bf16> (src/dispatch.rs:135-164)."""
    _fields_ = [("m", _size), ("k", _size), ("n", _size), ("alpha", _u16), ("a", _vp),
                ("rsa", _sdiff), ("csa", _sdiff), ("b", _vp), ("rsb", _sdiff), ("csb", _sdiff),
                ("beta", _u16), ("c", _vp), ("rsc", _sdiff), ("csc", _sdiff)]


class BatchProblemF32C(C.Structure):
    """``gk_batch_problem_f32``: BatchProblem<f32> (src/api/batched.rs:723-735)."""
    _fields_ = [("alpha", _f32), ("a", MatRefC), ("b", MatRefC), ("beta", _f32),
                ("c", MatMutC)]


class BatchProblemBf16C(C.Structure):
    """``gk_batch_problem_bf16``: BatchProblem<bf16> (src/api/batched.rs:723-735)."""
    _fields_ = [("alpha", _u16), ("a", MatRefC), ("b", MatRefC), ("beta", _u16),
                ("c", MatMutC)]


_REF = C.POINTER(MatRefC)
_MUT = C.POINTER(MatMutC)
_REQ = C.POINTER(RequantizeC)
_BIAS = C.POINTER(BiasC)

# name -> (restype, argtypes); one line per symbol of include/gemmkit_hip.h
SIGNATURES: dict[str, tuple] = {
    "gk_last_error": (C.c_char_p, []),
    "gk_version": (C.c_char_p, []),
    "gk_debug_plan": (C.c_int, [C.c_int32, C.c_int32, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                C.c_int64, C.POINTER(C.c_int32), C.POINTER(C.c_int64),
                                C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                C.POINTER(C.c_int32)]),
    "gk_init": (C.c_int, []),
    "gk_set_stream": (C.c_int, [_vp]),
    "gk_get_stream": (_vp, []),
    "gk_set_synchronous": (C.c_int, [C.c_int]),
    "gk_workspace_new": (_vp, []),
    "gk_workspace_with_capacity": (_vp, [_size]),
    "gk_workspace_free": (None, [_vp]),
    "gk_workspace_bytes": (_size, [_vp]),
    "gk_gemm_f32": (C.c_int, [_vp, _f32, _REF, _REF, _f32, _MUT, _u32]),
    "gk_gemm_f32_unchecked": (C.c_int, [_vp, _size, _size, _size, _f32, _vp, _sdiff, _sdiff,
                                        _vp, _sdiff, _sdiff, _f32, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_bf16": (C.c_int, [_vp, _u16, _REF, _REF, _u16, _MUT, _u32]),
    "gk_gemm_bf16_unchecked": (C.c_int, [_vp, _size, _size, _size, _u16, _vp, _sdiff, _sdiff,
                                         _vp, _sdiff, _sdiff, _u16, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_bf16_f32out": (C.c_int, [_vp, _f32, _REF, _REF, _f32, _MUT, _u32]),
    "gk_gemm_bf16_f32out_unchecked": (C.c_int, [_vp, _size, _size, _size, _f32, _vp, _sdiff,
                                                _sdiff, _vp, _sdiff, _sdiff, _f32, _vp, _sdiff,
                                                _sdiff, _u32]),
    "gk_gemm_i8": (C.c_int, [_vp, _i32, _REF, _REF, _i32, _MUT, _u32]),
    "gk_gemm_i8_unchecked": (C.c_int, [_vp, _size, _size, _size, _i32, _vp, _sdiff, _sdiff,
                                       _vp, _sdiff, _sdiff, _i32, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_i8_unchecked_noalloc": (C.c_int, [_size, _size, _size, _i32, _vp, _sdiff, _sdiff,
                                               _vp, _sdiff, _sdiff, _i32, _vp, _sdiff, _sdiff,
                                               _u32]),
    "gk_gemm_i8_requant": (C.c_int, [_vp, _REF, _REF, _REQ, _MUT, _u32]),
    "gk_gemm_i8_requant_u8": (C.c_int, [_vp, _REF, _REF, _REQ, _MUT, _u32]),
    "gk_gemm_i8_requant_unchecked": (C.c_int, [_vp, _size, _size, _size, _vp, _sdiff, _sdiff,
                                               _vp, _sdiff, _sdiff, _f32, _vp, _u8, _i32, _vp,
                                               _u8, _vp, _sdiff, _sdiff, _u32, _i32, _i32]),
    "gk_gemm_i8_requant_u8_unchecked": (C.c_int, [_vp, _size, _size, _size, _vp, _sdiff, _sdiff,
                                                  _vp, _sdiff, _sdiff, _f32, _vp, _u8, _i32, _vp,
                                                  _u8, _vp, _sdiff, _sdiff, _u32, _i32, _i32]),
    "gk_prepack_rhs_i8": (C.c_int, [_REF, C.POINTER(_vp)]),
    "gk_prepack_rhs_i8_unchecked": (C.c_int, [_vp, _sdiff, _sdiff, _size, _size, C.POINTER(_vp)]),
    "gk_packed_rhs_free": (None, [_vp]),
    "gk_packed_rhs_rows": (_size, [_vp]),
    "gk_packed_rhs_cols": (_size, [_vp]),
    "gk_gemm_i8_packed_b": (C.c_int, [_vp, _i32, _REF, _vp, _i32, _MUT, _u32]),
    "gk_gemm_i8_packed_b_unchecked": (C.c_int, [_vp, _i32, _size, _vp, _sdiff, _sdiff, _vp,
                                                _i32, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_i8_packed_b_requant": (C.c_int, [_vp, _REF, _vp, _REQ, _MUT, _u32]),
    "gk_gemm_i8_packed_b_requant_u8": (C.c_int, [_vp, _REF, _vp, _REQ, _MUT, _u32]),
    "gk_gemm_i8_packed_b_requant_unchecked": (C.c_int, [_vp, _size, _vp, _sdiff, _sdiff, _vp, _f32,
                                                        _vp, _u8, _i32, _vp, _u8, _vp, _sdiff,
                                                        _sdiff, _u32, _i32, _i32]),
    "gk_gemm_i8_packed_b_requant_u8_unchecked": (C.c_int, [_vp, _size, _vp, _sdiff, _sdiff, _vp,
                                                           _f32, _vp, _u8, _i32, _vp, _u8, _vp,
                                                           _sdiff, _sdiff, _u32, _i32, _i32]),
    "gk_gemm_batched_f32": (C.c_int, [_vp, _size, _f32, _REF, _sdiff, _REF, _sdiff, _f32, _MUT,
                                      _sdiff, _u32]),
    "gk_gemm_batched_f32_unchecked": (C.c_int, [_vp, _size, _size, _size, _size, _f32, _vp,
                                                _sdiff, _sdiff, _sdiff, _vp, _sdiff, _sdiff,
                                                _sdiff, _f32, _vp, _sdiff, _sdiff, _sdiff, _u32]),
    "gk_gemm_batched_bf16": (C.c_int, [_vp, _size, _u16, _REF, _sdiff, _REF, _sdiff, _u16, _MUT,
                                       _sdiff, _u32]),
    "gk_gemm_batched_bf16_unchecked": (C.c_int, [_vp, _size, _size, _size, _size, _u16, _vp,
                                                 _sdiff, _sdiff, _sdiff, _vp, _sdiff, _sdiff,
                                                 _sdiff, _u16, _vp, _sdiff, _sdiff, _sdiff, _u32]),
    "gk_gemm_batched_bf16_f32out": (C.c_int, [_vp, _size, _f32, _REF, _sdiff, _REF, _sdiff, _f32,
                                              _MUT, _sdiff, _u32]),
    "gk_gemm_batched_bf16_f32out_unchecked": (C.c_int, [_vp, _size, _size, _size, _size, _f32,
                                                        _vp, _sdiff, _sdiff, _sdiff, _vp, _sdiff,
                                                        _sdiff, _sdiff, _f32, _vp, _sdiff, _sdiff,
                                                        _sdiff, _u32]),
    "gk_gemm_batched_ptr_f32_unchecked": (C.c_int, [_vp, C.POINTER(ProblemF32C), _size, _u32]),
    "gk_gemm_batched_ptr_bf16_unchecked": (C.c_int, [_vp, C.POINTER(ProblemBf16C), _size, _u32]),
    "gk_gemm_batched_slice_f32": (C.c_int, [_vp, C.POINTER(BatchProblemF32C), _size, _u32]),
    "gk_gemm_batched_slice_bf16": (C.c_int, [_vp, C.POINTER(BatchProblemBf16C), _size, _u32]),
    "gk_prepack_rhs_f32": (C.c_int, [_REF, C.POINTER(_vp)]),
    "gk_prepack_rhs_f32_unchecked": (C.c_int, [_vp, _sdiff, _sdiff, _size, _size,
                                               C.POINTER(_vp)]),
    "gk_prepack_rhs_bf16": (C.c_int, [_REF, C.POINTER(_vp)]),
    "gk_prepack_rhs_bf16_unchecked": (C.c_int, [_vp, _sdiff, _sdiff, _size, _size,
                                                C.POINTER(_vp)]),
    "gk_prepack_lhs_f32": (C.c_int, [_REF, C.POINTER(_vp)]),
    "gk_prepack_lhs_f32_unchecked": (C.c_int, [_vp, _sdiff, _sdiff, _size, _size,
                                               C.POINTER(_vp)]),
    "gk_prepack_lhs_bf16": (C.c_int, [_REF, C.POINTER(_vp)]),
    "gk_prepack_lhs_bf16_unchecked": (C.c_int, [_vp, _sdiff, _sdiff, _size, _size,
                                                C.POINTER(_vp)]),
    "gk_packed_lhs_free": (None, [_vp]),
    "gk_packed_lhs_rows": (_size, [_vp]),
    "gk_packed_lhs_cols": (_size, [_vp]),
    "gk_gemm_packed_a_f32": (C.c_int, [_vp, _f32, _vp, _REF, _f32, _MUT, _u32]),
    "gk_gemm_packed_a_bf16": (C.c_int, [_vp, _u16, _vp, _REF, _u16, _MUT, _u32]),
    "gk_gemm_packed_a_f32_unchecked": (C.c_int, [_vp, _f32, _vp, _size, _vp, _sdiff, _sdiff,
                                                 _f32, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_packed_a_bf16_unchecked": (C.c_int, [_vp, _u16, _vp, _size, _vp, _sdiff, _sdiff,
                                                  _u16, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_packed_a_fused_f32": (C.c_int, [_vp, _f32, _vp, _REF, _f32, _MUT, _BIAS, _i32, _f32,
                                             _u32]),
    "gk_gemm_packed_a_fused_bf16": (C.c_int, [_vp, _u16, _vp, _REF, _u16, _MUT, _BIAS, _i32,
                                              _u16, _u32]),
    "gk_gemm_packed_a_fused_f32_unchecked": (C.c_int, [_vp, _f32, _vp, _size, _vp, _sdiff, _sdiff,
                                                       _f32, _vp, _sdiff, _sdiff, _vp, _i32, _u8,
                                                       _i32, _f32, _u32]),
    "gk_gemm_packed_a_fused_bf16_unchecked": (C.c_int, [_vp, _u16, _vp, _size, _vp, _sdiff,
                                                        _sdiff, _u16, _vp, _sdiff, _sdiff, _vp,
                                                        _i32, _u8, _i32, _u16, _u32]),
    "gk_gemm_packed_b_f32": (C.c_int, [_vp, _f32, _REF, _vp, _f32, _MUT, _u32]),
    "gk_gemm_packed_b_f32_unchecked": (C.c_int, [_vp, _f32, _size, _vp, _sdiff, _sdiff, _vp,
                                                 _f32, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_packed_b_bf16": (C.c_int, [_vp, _u16, _REF, _vp, _u16, _MUT, _u32]),
    "gk_gemm_packed_b_bf16_unchecked": (C.c_int, [_vp, _u16, _size, _vp, _sdiff, _sdiff, _vp,
                                                  _u16, _vp, _sdiff, _sdiff, _u32]),
    "gk_gemm_fused_f32": (C.c_int, [_vp, _f32, _REF, _REF, _f32, _MUT, _BIAS, _i32, _f32, _u32]),
    "gk_gemm_fused_bf16": (C.c_int, [_vp, _u16, _REF, _REF, _u16, _MUT, _BIAS, _i32, _u16,
                                     _u32]),
    "gk_gemm_fused_f32_unchecked": (C.c_int, [_vp, _size, _size, _size, _f32, _vp, _sdiff,
                                              _sdiff, _vp, _sdiff, _sdiff, _f32, _vp, _sdiff,
                                              _sdiff, _vp, _i32, _u8, _i32, _f32, _u32]),
    "gk_gemm_fused_bf16_unchecked": (C.c_int, [_vp, _size, _size, _size, _u16, _vp, _sdiff,
                                               _sdiff, _vp, _sdiff, _sdiff, _u16, _vp, _sdiff,
                                               _sdiff, _vp, _i32, _u8, _i32, _u16, _u32]),
    "gk_gemm_batched_fused_f32": (C.c_int, [_vp, _size, _f32, _REF, _sdiff, _REF, _sdiff, _f32,
                                            _MUT, _sdiff, _BIAS, _i32, _f32, _u32]),
    "gk_gemm_batched_fused_bf16": (C.c_int, [_vp, _size, _u16, _REF, _sdiff, _REF, _sdiff, _u16,
                                             _MUT, _sdiff, _BIAS, _i32, _u16, _u32]),
    "gk_gemm_batched_fused_f32_unchecked": (C.c_int, [_vp, _size, _size, _size, _size, _f32, _vp,
                                                      _sdiff, _sdiff, _sdiff, _vp, _sdiff, _sdiff,
                                                      _sdiff, _f32, _vp, _sdiff, _sdiff, _sdiff,
                                                      _vp, _i32, _u8, _i32, _f32, _u32]),
    "gk_gemm_batched_fused_bf16_unchecked": (C.c_int, [_vp, _size, _size, _size, _size, _u16,
                                                       _vp, _sdiff, _sdiff, _sdiff, _vp, _sdiff,
                                                       _sdiff, _sdiff, _u16, _vp, _sdiff, _sdiff,
                                                       _sdiff, _vp, _i32, _u8, _i32, _u16, _u32]),
    "gk_gemm_packed_b_fused_f32": (C.c_int, [_vp, _f32, _REF, _vp, _f32, _MUT, _BIAS, _i32, _f32,
                                             _u32]),
    "gk_gemm_packed_b_fused_bf16": (C.c_int, [_vp, _u16, _REF, _vp, _u16, _MUT, _BIAS, _i32,
                                              _u16, _u32]),
    "gk_gemm_packed_b_fused_f32_unchecked": (C.c_int, [_vp, _f32, _size, _vp, _sdiff, _sdiff,
                                                       _vp, _f32, _vp, _sdiff, _sdiff, _vp, _i32,
                                                       _u8, _i32, _f32, _u32]),
    "gk_gemm_packed_b_fused_bf16_unchecked": (C.c_int, [_vp, _u16, _size, _vp, _sdiff, _sdiff,
                                                        _vp, _u16, _vp, _sdiff, _sdiff, _vp,
                                                        _i32, _u8, _i32, _u16, _u32]),
}

_LIB: C.CDLL | None = None


class LibraryMissing(ImportError):
    pass


def lib() -> C.CDLL:
    """The loaded HIP library with typed signatures; raises when it is not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def last_error() -> str:
    return lib().gk_last_error().decode("utf-8", "replace")
