"""The oracle: CPU restatements of gemmkit's GEMM semantics.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or, for ``cpu_port``, as the timed CPU baseline).  The product path in
``gemmkit_amd`` never imports it and fails loudly when its HIP library is
missing.

Two shared libraries back it, both built by ``oracle/Makefile`` with gcc:

* ``liboracle.so`` (``oracle.c``) -- closed forms: the exact i8 GEMM
  (wrapping i32), the requantize map, bf16 RNE narrowing, f64 GEMM/GEMV,
  the seeded generators of gemmkit's tests.
* ``libcpu_port.so`` (``cpu_port.c``) -- the BLIS + AVX-512 VNNI restatement of
  gemmkit's CPU i8 path, timed as the CPU baseline.

Every wrapper takes and returns numpy arrays; strides are in elements.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict[str, C.CDLL] = {}


def build() -> None:
    """Compile the oracle libraries with gcc (idempotent)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _lib(name: str) -> C.CDLL:
    if name not in _LIBS:
        path = os.path.join(_HERE, name)
        if not os.path.exists(path):
            build()
        _LIBS[name] = C.CDLL(path)
    return _LIBS[name]


_i8p = C.POINTER(C.c_int8)
_u8p = C.POINTER(C.c_uint8)
_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_u16p = C.POINTER(C.c_uint16)
_sz = C.c_size_t
_sd = C.c_ssize_t


def _ptr(arr: np.ndarray, ty, offset: int = 0):
    """Pointer to element ``offset`` of a contiguous numpy buffer."""
    assert arr.flags["C_CONTIGUOUS"]
    return C.cast(arr.ctypes.data + offset * arr.itemsize, ty)


def _oracle() -> C.CDLL:
    lib = _lib("liboracle.so")
    if not getattr(lib, "_typed", False):
        lib.or_rng_next.restype = C.c_uint64
        lib.or_rng_next.argtypes = [C.POINTER(C.c_uint64)]
        for fn, ty in (("or_fill_i8_sym127", _i8p), ("or_fill_i8_full", _i8p),
                       ("or_rand_i8_100", _i8p), ("or_rand_vec_f64", _f64p),
                       ("or_rng_unit_f64", _f64p), ("or_rng_normal_f64", _f64p)):
            getattr(lib, fn).argtypes = [C.c_uint64, _sz, ty]
            getattr(lib, fn).restype = None
        lib.or_gemm_i8.argtypes = [_sz, _sz, _sz, C.c_int32, _i8p, _sd, _sd, _i8p, _sd, _sd,
                                   C.c_int32, _i32p, _sd, _sd]
        lib.or_gemm_i8.restype = None
        lib.or_round_ne_f64.argtypes = [C.c_double]
        lib.or_round_ne_f64.restype = C.c_double
        lib.or_requant_one.argtypes = [C.c_int32, C.c_int32, C.c_float, C.c_int32,
                                       C.c_int32, C.c_int32]
        lib.or_requant_one.restype = C.c_int32
        lib.or_gemm_i8_requant.argtypes = [_sz, _sz, _sz, _i8p, _sd, _sd, _i8p, _sd, _sd,
                                           C.c_float, _f32p, C.c_int32, _i32p, C.c_int,
                                           C.c_int32, C.c_int32, _u8p, _sd, _sd]
        lib.or_gemm_i8_requant.restype = None
        lib.or_requant_map.argtypes = [_sz, _sz, _i32p, _sd, _sd, C.c_float, _f32p, C.c_int32,
                                       _i32p, C.c_int, C.c_int32, C.c_int32, _u8p, _sd, _sd]
        lib.or_requant_map.restype = None
        lib.or_bf16_from_f32.argtypes = [C.c_float]
        lib.or_bf16_from_f32.restype = C.c_uint16
        lib.or_bf16_from_f32_n.argtypes = [_f32p, _sz, _u16p]
        lib.or_bf16_from_f32_n.restype = None
        lib.or_gemm_f64.argtypes = [_sz, _sz, _sz, C.c_double, _f32p, _sd, _sd, _f32p, _sd,
                                    _sd, C.c_double, _f32p, _sd, _sd, _f64p]
        lib.or_gemm_f64.restype = None
        lib.or_gemv_f64.argtypes = [_sz, _sz, C.c_double, _f32p, _sd, _sd, _f32p, _sd,
                                    C.c_double, _f32p, _sd, _f64p]
        lib.or_gemv_f64.restype = None
        lib.or_colsum_i32.argtypes = [_sz, _sz, _i32p, _sd, _sd, _i64p]
        lib.or_colsum_i32.restype = None
        lib.or_abft_i8.argtypes = [_sz, _sz, _sz, _i8p, _sd, _sd, _i8p, _sd, _sd, _i64p]
        lib.or_abft_i8.restype = None
        lib.or_fused_map_f32.argtypes = [_sz, _sz, _f32p, _sd, _sd, _f32p, C.c_int, C.c_int,
                                         C.c_float, _f32p, _sd, _sd]
        lib.or_fused_map_f32.restype = None
        lib.or_fused_map_bf16.argtypes = [_sz, _sz, _f32p, _sd, _sd, _u16p, C.c_int, C.c_int,
                                          C.c_uint16, _u16p, _sd, _sd]
        lib.or_fused_map_bf16.restype = None
        lib._typed = True
    return lib


# ----------------------------------------------------------------- generators

def rng_i8_sym127(seed: int, n: int) -> np.ndarray:
    """``make_i8`` (tests/epilogue/requant.rs:25-30): i8 in [-127, 127]."""
    out = np.empty(n, np.int8)
    _oracle().or_fill_i8_sym127(seed, n, _ptr(out, _i8p))
    return out


def rng_i8_full(seed: int, n: int) -> np.ndarray:
    """Rng (tests/epilogue/common.rs:16-34) ``next_u64() % 256 - 128``: full i8 range."""
    out = np.empty(n, np.int8)
    _oracle().or_fill_i8_full(seed, n, _ptr(out, _i8p))
    return out


def rand_i8_100(seed: int, n: int) -> np.ndarray:
    """``rand_i8`` (tests/correctness/common.rs:137-147): i8 in [-100, 100]."""
    out = np.empty(n, np.int8)
    _oracle().or_rand_i8_100(seed, n, _ptr(out, _i8p))
    return out


def rand_vec(seed: int, n: int) -> np.ndarray:
    """``rand_vec`` (tests/oracle_common/mod.rs:121-132): f64 uniform in [-1, 1)."""
    out = np.empty(n, np.float64)
    _oracle().or_rand_vec_f64(seed, n, _ptr(out, _f64p))
    return out


def rng_unit(seed: int, n: int) -> np.ndarray:
    """``Rng::unit`` (tests/epilogue/common.rs:30-33): f64 uniform in [-1, 1)."""
    out = np.empty(n, np.float64)
    _oracle().or_rng_unit_f64(seed, n, _ptr(out, _f64p))
    return out


def rng_normal(seed: int, n: int) -> np.ndarray:
    """Standard normals (Box-Muller over the Rng stream)."""
    out = np.empty(n, np.float64)
    _oracle().or_rng_normal_f64(seed, n, _ptr(out, _f64p))
    return out


def rng_next_u64(seed: int, count: int) -> list[int]:
    st = C.c_uint64(seed | 1)
    return [_oracle().or_rng_next(C.byref(st)) for _ in range(count)]


# --------------------------------------------------------------- closed forms

def gemm_i8(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc,
            a_off=0, b_off=0, c_off=0) -> None:
    """Exact strided i8 -> i32 GEMM, in place on ``c`` (oracle.c ``or_gemm_i8``)."""
    _oracle().or_gemm_i8(m, k, n, int(alpha), _ptr(a, _i8p, a_off), rsa, csa,
                         _ptr(b, _i8p, b_off), rsb, csb, int(beta),
                         _ptr(c, _i32p, c_off), rsc, csc)


def requant_one(acc, bias, scale, zp, lo=-128, hi=127) -> int:
    return _oracle().or_requant_one(int(acc), int(bias), float(scale), int(zp), lo, hi)


def round_ne_f64(x: float) -> float:
    return _oracle().or_round_ne_f64(float(x))


def gemm_i8_requant(m, k, n, a, rsa, csa, b, rsb, csb, scale, scales, zp, bias, axis,
                    lo, hi, c, rsc, csc) -> None:
    """Exact requantizing GEMM into the byte buffer ``c`` (int8 or uint8 numpy)."""
    lib = _oracle()
    sp = _ptr(np.ascontiguousarray(scales, np.float32), _f32p) if scales is not None else None
    bp = _ptr(np.ascontiguousarray(bias, np.int32), _i32p) if bias is not None else None
    keep = (scales, bias)  # noqa: F841 -- hold buffers for the call
    lib.or_gemm_i8_requant(m, k, n, _ptr(a, _i8p), rsa, csa, _ptr(b, _i8p), rsb, csb,
                           float(scale), sp, int(zp), bp, int(axis), int(lo), int(hi),
                           C.cast(c.ctypes.data, _u8p), rsc, csc)


def requant_map(m, n, acc, ra, ca, scale, scales, zp, bias, axis, lo, hi, c, rc, cc) -> None:
    """Requant map over an existing i32 accumulator matrix into byte buffer ``c``."""
    sp = _ptr(np.ascontiguousarray(scales, np.float32), _f32p) if scales is not None else None
    bp = _ptr(np.ascontiguousarray(bias, np.int32), _i32p) if bias is not None else None
    keep = (scales, bias)  # noqa: F841
    _oracle().or_requant_map(m, n, _ptr(acc, _i32p), ra, ca, float(scale), sp, int(zp), bp,
                             int(axis), int(lo), int(hi), C.cast(c.ctypes.data, _u8p), rc, cc)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, RNE with gemmkit's NaN rule."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    _oracle().or_bf16_from_f32_n(_ptr(x, _f32p), x.size, _ptr(out, _u16p))
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def gemm_f64(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta=0.0, c0=None, rsc=0, csc=0):
    """f64 closed form; returns a dense row-major (m, n) float64 array."""
    out = np.empty((m, n), np.float64)
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    cp = None
    if c0 is not None:
        c0 = np.ascontiguousarray(c0, np.float32)
        cp = _ptr(c0, _f32p)
    _oracle().or_gemm_f64(m, k, n, float(alpha), _ptr(a, _f32p), rsa, csa, _ptr(b, _f32p),
                          rsb, csb, float(beta), cp, rsc, csc, _ptr(out, _f64p))
    return out


def gemv_f64(rows, k, alpha, a, rs, cs, x, xs, beta=0.0, y0=None, ys=1):
    out = np.empty(rows, np.float64)
    a = np.ascontiguousarray(a, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    yp = None
    if y0 is not None:
        y0 = np.ascontiguousarray(y0, np.float32)
        yp = _ptr(y0, _f32p)
    _oracle().or_gemv_f64(rows, k, float(alpha), _ptr(a, _f32p), rs, cs, _ptr(x, _f32p), xs,
                          float(beta), yp, ys, _ptr(out, _f64p))
    return out


def colsum_i32(m, n, c, rsc, csc) -> np.ndarray:
    out = np.empty(n, np.int64)
    _oracle().or_colsum_i32(m, n, _ptr(c, _i32p), rsc, csc, _ptr(out, _i64p))
    return out


def abft_i8(m, k, n, a, rsa, csa, b, rsb, csb) -> np.ndarray:
    """(column sums of A) x B in exact i64: the expected column sums of A*B."""
    out = np.empty(n, np.int64)
    _oracle().or_abft_i8(m, k, n, _ptr(a, _i8p), rsa, csa, _ptr(b, _i8p), rsb, csb,
                         _ptr(out, _i64p))
    return out


def fused_map_f32(v: np.ndarray, bias=None, dim: int = 0, act: int = 0,
                  slope: float = 0.0) -> np.ndarray:
    """FusedEpi::apply (f32) over a 2-D float32 array; returns a new array."""
    v = np.ascontiguousarray(v, np.float32)
    m, n = v.shape
    out = np.empty_like(v)
    bp = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, np.float32)
        bp = _ptr(bias, _f32p)
    _oracle().or_fused_map_f32(m, n, _ptr(v, _f32p), n, 1, bp, int(dim), int(act),
                               float(slope), _ptr(out, _f32p), n, 1)
    return out


def fused_map_bf16(v: np.ndarray, bias_bits=None, dim: int = 0, act: int = 0,
                   slope_bits: int = 0) -> np.ndarray:
    """The bf16 fused map: f32 values in, bf16 bit patterns out (2-D)."""
    v = np.ascontiguousarray(v, np.float32)
    m, n = v.shape
    out = np.empty((m, n), np.uint16)
    bp = None
    if bias_bits is not None:
        bias_bits = np.ascontiguousarray(bias_bits, np.uint16)
        bp = _ptr(bias_bits, _u16p)
    _oracle().or_fused_map_bf16(m, n, _ptr(v, _f32p), n, 1, bp, int(dim), int(act),
                                int(slope_bits), _ptr(out, _u16p), n, 1)
    return out


# ------------------------------------------------------------------ CPU port

def _port() -> C.CDLL:
    lib = _lib("libcpu_port.so")
    if not getattr(lib, "_typed", False):
        vp = C.c_void_p
        f32p = C.POINTER(C.c_float)
        u16p = C.POINTER(C.c_uint16)
        u8p = C.POINTER(C.c_uint8)
        lib.port_gemm_i8.argtypes = [_sz, _sz, _sz, C.c_int32, _i8p, _sd, _sd, _i8p, _sd, _sd,
                                     C.c_int32, _i32p, _sd, _sd, C.c_int]
        lib.port_gemm_i8.restype = C.c_int
        lib.port_prepack_b_i8.argtypes = [_sz, _sz, _i8p, _sd, _sd, C.c_int]
        lib.port_prepack_b_i8.restype = vp
        lib.port_packed_b_free.argtypes = [vp]
        lib.port_packed_b_free.restype = None
        lib.port_gemm_i8_requant.argtypes = [_sz, _sz, _sz, _i8p, _sd, _sd, _i8p, _sd, _sd, vp,
                                             C.c_float, f32p, C.c_int32, _i32p, C.c_int,
                                             C.c_int32, C.c_int32, u8p, _sd, _sd, C.c_int]
        lib.port_gemm_i8_requant.restype = C.c_int
        lib.port_gemm_f32.argtypes = [_sz, _sz, _sz, C.c_float, f32p, _sd, _sd, f32p, _sd, _sd,
                                      C.c_float, f32p, _sd, _sd, C.c_int]
        lib.port_gemm_f32.restype = C.c_int
        lib.port_gemm_batched_bf16_f32out.argtypes = [_sz, _sz, _sz, _sz, C.c_float, u16p, _sd,
                                                      _sd, _sd, u16p, _sd, _sd, _sd, C.c_float,
                                                      f32p, _sd, _sd, _sd, C.c_int]
        lib.port_gemm_batched_bf16_f32out.restype = C.c_int
        lib.port_gemv_f32.argtypes = [_sz, _sz, C.c_float, f32p, _sd, f32p, C.c_float, f32p,
                                      _sd, C.c_int]
        lib.port_gemv_f32.restype = C.c_int
        for name in ("port_has_vnni", "port_has_avx512f", "port_has_bf16", "port_max_threads"):
            getattr(lib, name).restype = C.c_int
        lib._typed = True
    return lib


def port_gemm_i8(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc,
                 threads: int = 0) -> int:
    """gemmkit's CPU i8 path restated (BLIS + VNNI); returns the thread count used."""
    return _port().port_gemm_i8(m, k, n, int(alpha), _ptr(a, _i8p), rsa, csa, _ptr(b, _i8p),
                                rsb, csb, int(beta), _ptr(c, _i32p), rsc, csc, int(threads))


class PortPackedB:
    """A B operand packed once in the VNNI panel layout (port_prepack_b_i8)."""

    def __init__(self, k, n, b, rsb, csb, threads: int = 0):
        self._keep = b
        self.k, self.n = k, n
        self.h = _port().port_prepack_b_i8(k, n, _ptr(b, _i8p), rsb, csb, int(threads))

    def __del__(self):
        h, self.h = getattr(self, "h", None), None
        if h:
            _port().port_packed_b_free(h)


def port_gemm_i8_requant(m, k, n, a, rsa, csa, b, rsb, csb, scale, scales, zp, bias, axis,
                         lo, hi, c, rsc, csc, threads: int = 0, packed: PortPackedB = None) -> int:
    """gemmkit's requantizing VNNI path restated (kc = k, map per drained tile);
    `packed` replaces b.  Same argument meaning as gemm_i8_requant below."""
    f32p = C.POINTER(C.c_float)
    return _port().port_gemm_i8_requant(
        m, k, n, _ptr(a, _i8p), rsa, csa, None if packed is not None else _ptr(b, _i8p), rsb,
        csb, packed.h if packed is not None else None, float(scale),
        None if scales is None else _ptr(scales, f32p), int(zp),
        None if bias is None else _ptr(bias, _i32p), int(axis), int(lo), int(hi),
        _ptr(c, C.POINTER(C.c_uint8)), rsc, csc, int(threads))


def port_gemm_f32(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc,
                  threads: int = 0) -> int:
    """gemmkit's f32 path restated (BLIS + AVX-512F 32x12 FMA microtile)."""
    f32p = C.POINTER(C.c_float)
    return _port().port_gemm_f32(m, k, n, float(alpha), _ptr(a, f32p), rsa, csa, _ptr(b, f32p),
                                 rsb, csb, float(beta), _ptr(c, f32p), rsc, csc, int(threads))


def port_gemm_batched_bf16_f32out(batch, m, k, n, alpha, a_bits, rsa, csa, a_bs, b_bits, rsb,
                                  csb, b_bs, beta, c, rsc, csc, c_bs, threads: int = 0) -> int:
    """gemmkit's bf16 dot path (vdpbf16ps, f32 accumulation) over a batch, f32
    output; a_bits/b_bits are the bf16 bit patterns (uint16)."""
    f32p = C.POINTER(C.c_float)
    u16p = C.POINTER(C.c_uint16)
    return _port().port_gemm_batched_bf16_f32out(
        batch, m, k, n, float(alpha), _ptr(a_bits, u16p), rsa, csa, a_bs, _ptr(b_bits, u16p),
        rsb, csb, b_bs, float(beta), _ptr(c, f32p), rsc, csc, c_bs, int(threads))


def port_gemv_f32(rows, k, alpha, a, lda, x, beta, y, ys=1, threads: int = 0) -> int:
    """gemmkit's row-partitioned f32 GEMV (dot_rows) restated."""
    f32p = C.POINTER(C.c_float)
    return _port().port_gemv_f32(rows, k, float(alpha), _ptr(a, f32p), lda, _ptr(x, f32p),
                                 float(beta), _ptr(y, f32p), ys, int(threads))


def port_has_vnni() -> bool:
    return bool(_port().port_has_vnni())


def port_has_avx512f() -> bool:
    return bool(_port().port_has_avx512f())


def port_has_bf16() -> bool:
    return bool(_port().port_has_bf16())


def port_max_threads() -> int:
    return int(_port().port_max_threads())
