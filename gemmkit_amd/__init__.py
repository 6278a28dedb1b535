"""gemmkit_amd -- gemmkit's GEMM API on MI355X (gfx950) matrix cores.

Python mirror of the reference's Rust surface (gemmkit/src/lib.rs:98-148),
calling the hand-written HIP kernels of ``libgemmkit_hip.so`` through its C ABI
(``include/gemmkit_hip.h``).  Names, argument order and meaning follow the
reference:

===============================  ==============================================
reference (gemmkit/src/...)      here
===============================  ==============================================
``MatRef`` / ``MatMut``          :class:`MatRef` / :class:`MatMut` over a 1-D
  (api.rs:92-180)                device tensor (the "slice"), strides in elements
``gemm``, ``gemm_with``          :func:`gemm` (f32, bf16), ``ws=`` for ``_with``
``gemm_unchecked(_with)``        :func:`gemm_unchecked`
``gemm_i8(_with)``               :func:`gemm_i8`
``gemm_i8_unchecked(_with)``     :func:`gemm_i8_unchecked`
``gemm_i8_requant(_u8)``         :func:`gemm_i8_requant`, :func:`gemm_i8_requant_u8`
``..._requant_unchecked``        :func:`gemm_i8_requant_unchecked`
``prepack_rhs_i8``               :func:`prepack_rhs_i8` -> :class:`PackedRhs`
``gemm_i8_packed_b(_with)``      :func:`gemm_i8_packed_b`
``gemm_batched(_with)``          :func:`gemm_batched`
``prepack_rhs`` (f32, bf16)      :func:`prepack_rhs` -> :class:`PackedRhs`
``gemm_packed_b(_with)``         :func:`gemm_packed_b`, :func:`gemm_packed_b_unchecked`
``Bias`` / ``Activation``        :class:`Bias` / :class:`Activation`
  (api/fused.rs:17-31)
``gemm_fused(_with)``            :func:`gemm_fused`, :func:`gemm_fused_unchecked`
``gemm_batched_fused(_with)``    :func:`gemm_batched_fused`,
                                 :func:`gemm_batched_fused_unchecked`
``gemm_packed_b_fused(_with)``   :func:`gemm_packed_b_fused`,
                                 :func:`gemm_packed_b_fused_unchecked`
``Parallelism``                  :class:`Parallelism` (accepted, ignored: the
                                 device grid decides)
``Workspace``                    :class:`Workspace` (a device scratch arena)
===============================  ==============================================

Where the reference panics, these functions raise :class:`GemmkitError` with
the reference's message.  Extensions of this engine (no reference
counterpart): f32 output for bf16 GEMMs (:func:`gemm_bf16_f32out`,
:func:`gemm_batched_bf16_f32out`), per-column requant vectors
(``RequantScale.PerCol``, ``Requantize(bias_axis="col")``), a ReLU after
requantization (``Requantize(relu=True)``), and prepacked-B requantization
(:func:`gemm_i8_packed_b_requant`).

All tensors must live on the HIP device; calls are synchronous by default and
run on torch's current stream.  There is no CPU fallback: a missing library
raises.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence, Union

import torch

from . import _lib
from ._lib import BiasC, MatMutC, MatRefC, RequantizeC

__all__ = [
    "GemmkitError", "MatRef", "MatMut", "Parallelism", "Workspace", "RequantScale",
    "Requantize", "PackedRhs", "gemm", "gemm_unchecked", "gemm_bf16_f32out", "gemm_i8",
    "gemm_i8_unchecked", "gemm_i8_requant", "gemm_i8_requant_u8", "gemm_i8_requant_unchecked",
    "gemm_i8_requant_u8_unchecked", "prepack_rhs_i8", "gemm_i8_packed_b",
    "gemm_i8_packed_b_unchecked", "gemm_i8_packed_b_requant", "gemm_i8_packed_b_requant_u8",
    "gemm_i8_packed_b_requant_unchecked",
    "gemm_batched", "gemm_batched_unchecked", "gemm_batched_bf16_f32out", "prepack_rhs",
    "gemm_packed_b", "gemm_packed_b_unchecked", "Bias", "Activation", "gemm_fused",
    "gemm_fused_unchecked", "gemm_batched_fused", "gemm_batched_fused_unchecked",
    "gemm_packed_b_fused", "gemm_packed_b_fused_unchecked", "set_synchronous",
    "library_path", "version",
]

library_path = _lib.LIB_PATH


class GemmkitError(RuntimeError):
    """Raised where the reference panics; ``code`` is the C ABI's gk_status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def _check(rc: int) -> None:
    if rc != 0:
        raise GemmkitError(rc, _lib.last_error())


def version() -> str:
    return _lib.lib().gk_version().decode()


TILE_NAMES = {0: "256x256", 1: "256x128", 2: "128x128", 3: "64x64", 4: "256x256w8",
              5: "256x128o2", 6: "256x256k128", 7: "256x256w8k128", 8: "128x192k128",
              9: "128x96k128o2", 10: "256x384w8k128",
              11: "256x352w8k128", 12: "256x256w8m16", 13: "256x352w8m16"}
_IN_CODES = {"i8": 0, "bf16": 1, "f32": 2}
_KIND_CODES = {"i32": 0, "f32": 1, "bf16": 2, "q8": 3}


def debug_plan(in_type: str, kind: str, m: int, n: int, kbytes: int, batch: int = 1,
               pitches: bool = False, ld_b: int = 0):
    """Extension (no reference counterpart): the matrix-core launch plan the
    dispatcher would choose for an m x n product in the kernel frame with
    `kbytes` bytes of K per row (and B^T rows `ld_b` bytes apart, 0 for
    packed rows), as (tile, na, tile_b): na > 0 means a second launch covers
    columns [na, n) with tile_b.  pitches=True: (tile, pitch, na, tile_b,
    pitch_b), a pitch of 0 meaning the tile's width.  Host-only."""
    t, na, tb = C.c_int32(), C.c_int64(), C.c_int32()
    pa, pb = C.c_int32(), C.c_int32()
    _check(_lib.lib().gk_debug_plan(_IN_CODES[in_type], _KIND_CODES[kind], m, n, batch, kbytes,
                                    ld_b, C.byref(t), C.byref(na), C.byref(tb), C.byref(pa),
                                    C.byref(pb)))
    if pitches:
        return TILE_NAMES[t.value], pa.value, na.value, TILE_NAMES[tb.value], pb.value
    return TILE_NAMES[t.value], na.value, TILE_NAMES[tb.value]


def set_synchronous(on: bool) -> None:
    """True (default): every call waits for its kernels, like the reference."""
    _lib.lib().gk_set_synchronous(1 if on else 0)


def _bind_stream() -> None:
    L = _lib.lib()
    if not torch.cuda.is_available():
        raise GemmkitError(-7, "gemmkit_amd: no HIP device available; tensors must live on "
                               "the HIP device")
    s = torch.cuda.current_stream().cuda_stream
    L.gk_set_stream(C.c_void_p(s))


# ---------------------------------------------------------------------- types

class Parallelism:
    """Parallelism (src/parallel.rs:25): ``Serial`` or ``Rayon(n)`` (0 = all)."""

    def __init__(self, threads: int):
        self.threads = int(threads)

    @staticmethod
    def Rayon(n: int) -> "Parallelism":  # noqa: N802 -- mirrors the Rust variant
        return Parallelism(n)

    def __repr__(self) -> str:
        return "Serial" if self.threads == 1 else f"Rayon({self.threads})"


Parallelism.Serial = Parallelism(1)  # type: ignore[attr-defined]


def _par(par: Optional[Parallelism]) -> int:
    return 1 if par is None else par.threads


class Workspace:
    """Workspace (src/workspace.rs:53): a device scratch arena owned by the caller."""

    def __init__(self) -> None:
        L = _lib.lib()
        self._free = L.gk_workspace_free  # held so __del__ works during interpreter exit
        self._h = L.gk_workspace_new()

    @classmethod
    def with_capacity(cls, nbytes: int) -> "Workspace":
        """Workspace::with_capacity (src/workspace.rs:78): the arena allocated up
        front, so later calls (also under HIP graph capture) need not grow it."""
        L = _lib.lib()
        ws = cls.__new__(cls)
        ws._free = L.gk_workspace_free
        ws._h = L.gk_workspace_with_capacity(int(nbytes))
        if not ws._h:
            raise MemoryError(f"gemmkit: workspace allocation of {nbytes} bytes failed")
        return ws

    @property
    def handle(self):
        return self._h

    def bytes(self) -> int:
        return int(_lib.lib().gk_workspace_bytes(self._h))

    def __del__(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._free(h)


def _ws(ws: Optional[Workspace]):
    return None if ws is None else ws.handle


def _slice(data: torch.Tensor, what: str) -> torch.Tensor:
    if not isinstance(data, torch.Tensor):
        raise TypeError(f"gemmkit_amd: {what} data must be a torch.Tensor")
    if data.device.type != "cuda":
        raise GemmkitError(-7, f"gemmkit_amd: {what} data must live on the HIP device")
    if not data.is_contiguous():
        raise TypeError(f"gemmkit_amd: {what} data must be a contiguous slice")
    return data


class MatRef:
    """Immutable strided view (src/api.rs:92-140): element (i, j) at ``i*rs + j*cs``."""

    def __init__(self, data: torch.Tensor, rows: int, cols: int, rs: int, cs: int):
        self.data, self.rows, self.cols, self.rs, self.cs = data, int(rows), int(cols), int(rs), int(cs)

    @classmethod
    def from_row_major(cls, data, rows, cols):
        return cls(data, rows, cols, cols, 1)

    @classmethod
    def from_col_major(cls, data, rows, cols):
        return cls(data, rows, cols, 1, rows)

    def _c(self, dtype: torch.dtype, what: str) -> MatRefC:
        d = _slice(self.data, what)
        if d.dtype != dtype:
            raise TypeError(f"gemmkit_amd: {what} must be {dtype}, got {d.dtype}")
        return MatRefC(d.data_ptr(), d.numel(), self.rows, self.cols, self.rs, self.cs)


class MatMut(MatRef):
    """Mutable strided view (src/api.rs:107-180); the output C."""

    def _c(self, dtype: torch.dtype, what: str) -> MatMutC:  # type: ignore[override]
        d = _slice(self.data, what)
        if d.dtype != dtype:
            raise TypeError(f"gemmkit_amd: {what} must be {dtype}, got {d.dtype}")
        return MatMutC(d.data_ptr(), d.numel(), self.rows, self.cols, self.rs, self.cs)


def _bf16_bits(x: float) -> int:
    """f32 -> bf16 bit pattern, round to nearest even (NaN quieted)."""
    return int(torch.tensor([x], dtype=torch.float32).to(torch.bfloat16).view(torch.int16)
               .item()) & 0xFFFF


# ------------------------------------------------------------------ plain gemm

def gemm(alpha, a: MatRef, b: MatRef, beta, c: MatMut,
         par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm`` / ``gemm_with`` (src/api.rs:400-450): C <- alpha*A*B + beta*C.

    The element type follows the tensors: float32 or bfloat16 (f32 accumulation,
    one RNE narrowing; ``alpha``/``beta`` are rounded to bf16 like the
    reference's bf16 scalars)."""
    _bind_stream()
    L = _lib.lib()
    dt = a.data.dtype
    if dt == torch.float32:
        _check(L.gk_gemm_f32(_ws(ws), float(alpha), a._c(dt, "A"), b._c(dt, "B"), float(beta),
                             c._c(dt, "C"), _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_bf16(_ws(ws), _bf16_bits(alpha), a._c(dt, "A"), b._c(dt, "B"),
                              _bf16_bits(beta), c._c(dt, "C"), _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm supports float32 and bfloat16, got {dt}")


def gemm_bf16_f32out(alpha: float, a: MatRef, b: MatRef, beta: float, c: MatMut,
                     par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """Extension: bf16 inputs, f32 accumulation, f32 alpha/beta and output."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_bf16_f32out(_ws(ws), float(alpha), a._c(torch.bfloat16, "A"),
                                          b._c(torch.bfloat16, "B"), float(beta),
                                          c._c(torch.float32, "C"), _par(par)))


def _ptr(t: Optional[torch.Tensor], off: int = 0) -> Optional[int]:
    if t is None:
        return None
    return t.data_ptr() + off * t.element_size()


def gemm_unchecked(m, k, n, alpha, a: torch.Tensor, rsa, csa, b: torch.Tensor, rsb, csb, beta,
                   c: torch.Tensor, rsc, csc, par=None, ws=None, a_off=0, b_off=0, c_off=0):
    """``gemm_unchecked(_with)`` (src/api.rs:469-580): raw strides, no checks.

    ``*_off`` are element offsets of the base pointers (negative strides walk
    backwards from there, as the reference allows on this tier)."""
    _bind_stream()
    L = _lib.lib()
    if a.dtype == torch.float32:
        _check(L.gk_gemm_f32_unchecked(_ws(ws), m, k, n, float(alpha), _ptr(a, a_off), rsa, csa,
                                       _ptr(b, b_off), rsb, csb, float(beta), _ptr(c, c_off), rsc,
                                       csc, _par(par)))
    elif a.dtype == torch.bfloat16:
        _check(L.gk_gemm_bf16_unchecked(_ws(ws), m, k, n, _bf16_bits(alpha), _ptr(a, a_off), rsa,
                                        csa, _ptr(b, b_off), rsb, csb, _bf16_bits(beta),
                                        _ptr(c, c_off), rsc, csc, _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_unchecked supports float32 and bfloat16, got {a.dtype}")


# -------------------------------------------------------------------- i8 gemm

def gemm_i8(alpha: int, a: MatRef, b: MatRef, beta: int, c: MatMut,
            par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_i8`` / ``gemm_i8_with`` (src/api/int8.rs:22-73): wrapping i32."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8(_ws(ws), int(alpha), a._c(torch.int8, "A"),
                                 b._c(torch.int8, "B"), int(beta), c._c(torch.int32, "C"),
                                 _par(par)))


def gemm_i8_unchecked(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc, par=None,
                      ws=None, a_off=0, b_off=0, c_off=0) -> None:
    """``gemm_i8_unchecked(_with)`` (src/api/int8.rs:86-178)."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_unchecked(_ws(ws), m, k, n, int(alpha), _ptr(a, a_off), rsa,
                                           csa, _ptr(b, b_off), rsb, csb, int(beta),
                                           _ptr(c, c_off), rsc, csc, _par(par)))


# ------------------------------------------------------------------- requant

class RequantScale:
    """RequantScale (src/api/int8.rs:185-194): ``PerTensor(f)`` or ``PerRow(tensor)``;
    ``PerCol(tensor)`` is this engine's per-output-column extension."""

    def __init__(self, kind: str, value):
        self.kind, self.value = kind, value

    @staticmethod
    def PerTensor(s: float) -> "RequantScale":  # noqa: N802
        return RequantScale("tensor", float(s))

    @staticmethod
    def PerRow(s: torch.Tensor) -> "RequantScale":  # noqa: N802
        return RequantScale("row", s)

    @staticmethod
    def PerCol(s: torch.Tensor) -> "RequantScale":  # noqa: N802
        return RequantScale("col", s)


@dataclass
class Requantize:
    """Requantize (src/api/int8.rs:196-209).  ``bias`` is per row like the
    reference unless ``bias_axis="col"``; a per-column scale implies a per-column
    bias.  ``relu`` (extension) clamps the output below at the zero point."""
    scale: RequantScale
    zero_point: int = 0
    bias: Optional[torch.Tensor] = None
    bias_axis: str = "row"
    relu: bool = False

    def _c(self) -> RequantizeC:
        # One channel axis serves scales and bias, as the reference's bias_dim
        # does (src/dispatch/int.rs:640-660).
        if self.scale.kind == "row" and self.bias is not None and self.bias_axis == "col":
            raise GemmkitError(-4, "gemmkit_amd: per-row scales need a per-row bias")
        axis = 1 if (self.scale.kind == "col" or self.bias_axis == "col") else 0
        r = RequantizeC()
        if self.scale.kind == "tensor":
            r.scale, r.scales, r.scales_len = self.scale.value, None, 0
        else:
            s = _slice(self.scale.value, "requantize scales")
            if s.dtype != torch.float32:
                raise TypeError("gemmkit_amd: requantize scales must be float32")
            r.scale, r.scales, r.scales_len = 0.0, s.data_ptr(), s.numel()
        r.zero_point = int(self.zero_point)
        if self.bias is not None:
            bt = _slice(self.bias, "requantize bias")
            if bt.dtype != torch.int32:
                raise TypeError("gemmkit_amd: requantize bias must be int32")
            r.bias, r.bias_len = bt.data_ptr(), bt.numel()
        else:
            r.bias, r.bias_len = None, 0
        r.axis = axis
        r.act = 1 if self.relu else 0
        return r


def gemm_i8_requant(a: MatRef, b: MatRef, req: Requantize, c: MatMut,
                    par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_i8_requant(_with)`` (src/api/int8.rs:230-328): i8 out, [-128, 127]."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_requant(_ws(ws), a._c(torch.int8, "A"), b._c(torch.int8, "B"),
                                         C.byref(req._c()), c._c(torch.int8, "C"), _par(par)))


def gemm_i8_requant_u8(a: MatRef, b: MatRef, req: Requantize, c: MatMut,
                       par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_i8_requant_u8(_with)`` (src/api/int8.rs:479-555): u8 out, [0, 255]."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_requant_u8(_ws(ws), a._c(torch.int8, "A"),
                                            b._c(torch.int8, "B"), C.byref(req._c()),
                                            c._c(torch.uint8, "C"), _par(par)))


def gemm_i8_requant_unchecked(m, k, n, a, rsa, csa, b, rsb, csb, scale, row_scales, zero_point,
                              bias, c, rsc, csc, par=None, ws=None, axis=0, relu=False,
                              a_off=0, b_off=0, c_off=0) -> None:
    """``gemm_i8_requant_unchecked(_with)`` (src/api/int8.rs:347-457)."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_requant_unchecked(
        _ws(ws), m, k, n, _ptr(a, a_off), rsa, csa, _ptr(b, b_off), rsb, csb, float(scale),
        _ptr(row_scales), 1 if row_scales is not None else 0, int(zero_point), _ptr(bias),
        1 if bias is not None else 0, _ptr(c, c_off), rsc, csc, _par(par), int(axis),
        1 if relu else 0))


def gemm_i8_requant_u8_unchecked(m, k, n, a, rsa, csa, b, rsb, csb, scale, row_scales,
                                 zero_point, bias, c, rsc, csc, par=None, ws=None, axis=0,
                                 relu=False, a_off=0, b_off=0, c_off=0) -> None:
    """``gemm_i8_requant_u8_unchecked(_with)`` (src/api/int8.rs:562-672)."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_requant_u8_unchecked(
        _ws(ws), m, k, n, _ptr(a, a_off), rsa, csa, _ptr(b, b_off), rsb, csb, float(scale),
        _ptr(row_scales), 1 if row_scales is not None else 0, int(zero_point), _ptr(bias),
        1 if bias is not None else 0, _ptr(c, c_off), rsc, csc, _par(par), int(axis),
        1 if relu else 0))


# ---------------------------------------------------------------- prepacked B

class PackedRhs:
    """PackedRhs<T> (src/api/packed.rs:34-52): B packed once on the device
    (i8 from :func:`prepack_rhs_i8`, f32/bf16 from :func:`prepack_rhs`)."""

    def __init__(self, handle):
        self._free = _lib.lib().gk_packed_rhs_free  # held so __del__ works during interpreter exit
        self._h = handle

    @property
    def handle(self):
        return self._h

    def rows(self) -> int:
        return int(_lib.lib().gk_packed_rhs_rows(self._h))

    def cols(self) -> int:
        return int(_lib.lib().gk_packed_rhs_cols(self._h))

    def __del__(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._free(h)


def prepack_rhs_i8(b: MatRef) -> PackedRhs:
    """``prepack_rhs_i8`` (src/api/packed.rs:372-386)."""
    _bind_stream()
    out = C.c_void_p()
    _check(_lib.lib().gk_prepack_rhs_i8(b._c(torch.int8, "B"), C.byref(out)))
    return PackedRhs(out.value)


def gemm_i8_packed_b(alpha: int, a: MatRef, packed: PackedRhs, beta: int, c: MatMut,
                     par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_i8_packed_b(_with)`` (src/api/packed.rs:473-560): requires a
    column-major-ish C, like the reference."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_packed_b(_ws(ws), int(alpha), a._c(torch.int8, "A"),
                                          packed.handle, int(beta), c._c(torch.int32, "C"),
                                          _par(par)))


def gemm_i8_packed_b_unchecked(alpha, m, a, rsa, csa, packed: PackedRhs, beta, c, rsc, csc,
                               par=None, ws=None, a_off=0, c_off=0) -> None:
    """``gemm_i8_packed_b_unchecked(_with)`` (src/api/packed.rs:575-656)."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_packed_b_unchecked(_ws(ws), int(alpha), m, _ptr(a, a_off), rsa,
                                                    csa, packed.handle, int(beta),
                                                    _ptr(c, c_off), rsc, csc, _par(par)))


def gemm_i8_packed_b_requant(a: MatRef, packed: PackedRhs, req: Requantize, c: MatMut,
                             par: Optional[Parallelism] = None,
                             ws: Optional[Workspace] = None) -> None:
    """Extension: requantizing GEMM against a prepacked B (i8 out, any C layout)."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_packed_b_requant(_ws(ws), a._c(torch.int8, "A"), packed.handle,
                                                  C.byref(req._c()), c._c(torch.int8, "C"),
                                                  _par(par)))


def gemm_i8_packed_b_requant_u8(a: MatRef, packed: PackedRhs, req: Requantize, c: MatMut,
                                par: Optional[Parallelism] = None,
                                ws: Optional[Workspace] = None) -> None:
    """Extension: the u8-output twin of :func:`gemm_i8_packed_b_requant`."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_i8_packed_b_requant_u8(_ws(ws), a._c(torch.int8, "A"),
                                                     packed.handle, C.byref(req._c()),
                                                     c._c(torch.uint8, "C"), _par(par)))


def gemm_i8_packed_b_requant_unchecked(m, a, rsa, csa, packed: PackedRhs, scale, scales,
                                       zero_point, bias, c, rsc, csc, par=None, ws=None,
                                       axis=0, relu=False, u8=False, a_off=0, c_off=0) -> None:
    """Extension: unchecked prepacked-B requant (no validation, no host copies)."""
    _bind_stream()
    fn = (_lib.lib().gk_gemm_i8_packed_b_requant_u8_unchecked if u8
          else _lib.lib().gk_gemm_i8_packed_b_requant_unchecked)
    _check(fn(_ws(ws), m, _ptr(a, a_off), rsa, csa, packed.handle, float(scale), _ptr(scales),
              1 if scales is not None else 0, int(zero_point), _ptr(bias),
              1 if bias is not None else 0, _ptr(c, c_off), rsc, csc, _par(par), int(axis),
              1 if relu else 0))


# ------------------------------------------------------------------- batched

def gemm_batched(batch: int, alpha, a: MatRef, a_batch_stride: int, b: MatRef,
                 b_batch_stride: int, beta, c: MatMut, c_batch_stride: int,
                 par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_batched(_with)`` (src/api/batched.rs:188-283), float32 or bfloat16."""
    _bind_stream()
    L = _lib.lib()
    dt = a.data.dtype
    if dt == torch.float32:
        _check(L.gk_gemm_batched_f32(_ws(ws), batch, float(alpha), a._c(dt, "A"), a_batch_stride,
                                     b._c(dt, "B"), b_batch_stride, float(beta), c._c(dt, "C"),
                                     c_batch_stride, _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_batched_bf16(_ws(ws), batch, _bf16_bits(alpha), a._c(dt, "A"),
                                      a_batch_stride, b._c(dt, "B"), b_batch_stride,
                                      _bf16_bits(beta), c._c(dt, "C"), c_batch_stride, _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_batched supports float32 and bfloat16, got {dt}")


@dataclass
class GemmProblem:
    """GemmProblem (src/dispatch.rs:135-164): one independent product of the
    pointer-array batched form; a, b, c are device tensors (element offsets
    a_off, b_off, c_off), all float32 or all bfloat16."""
    m: int
    k: int
    n: int
    alpha: float
    a: torch.Tensor
    rsa: int
    csa: int
    b: torch.Tensor
    rsb: int
    csb: int
    beta: float
    c: torch.Tensor
    rsc: int
    csc: int
    a_off: int = 0
    b_off: int = 0
    c_off: int = 0


@dataclass
class BatchProblem:
    """BatchProblem (src/api/batched.rs:723-735): one element of gemm_batched_slice."""
    alpha: float
    a: MatRef
    b: MatRef
    beta: float
    c: MatMut


def gemm_batched_ptr_unchecked(problems, par: Optional[Parallelism] = None,
                               ws: Optional[Workspace] = None) -> None:
    """``gemm_batched_ptr_unchecked`` (src/api/batched.rs:711-720): every problem as the
    standalone gemm would run it; the outputs must be pairwise disjoint."""
    _bind_stream()
    if not problems:
        return
    L = _lib.lib()
    dt = problems[0].a.dtype
    if dt == torch.float32:
        arr = (_lib.ProblemF32C * len(problems))(*[
            _lib.ProblemF32C(p.m, p.k, p.n, float(p.alpha), _ptr(p.a, p.a_off), p.rsa, p.csa,
                             _ptr(p.b, p.b_off), p.rsb, p.csb, float(p.beta), _ptr(p.c, p.c_off),
                             p.rsc, p.csc) for p in problems])
        _check(L.gk_gemm_batched_ptr_f32_unchecked(_ws(ws), arr, len(problems), _par(par)))
    elif dt == torch.bfloat16:
        arr = (_lib.ProblemBf16C * len(problems))(*[
            _lib.ProblemBf16C(p.m, p.k, p.n, _bf16_bits(p.alpha), _ptr(p.a, p.a_off), p.rsa,
                              p.csa, _ptr(p.b, p.b_off), p.rsb, p.csb, _bf16_bits(p.beta),
                              _ptr(p.c, p.c_off), p.rsc, p.csc) for p in problems])
        _check(L.gk_gemm_batched_ptr_bf16_unchecked(_ws(ws), arr, len(problems), _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_batched_ptr_unchecked supports float32 and bfloat16")


def gemm_batched_slice(problems, par: Optional[Parallelism] = None,
                       ws: Optional[Workspace] = None) -> None:
    """``gemm_batched_slice`` (src/api/batched.rs:748-799): per-element shape, bounds and
    self-alias checks, then the pointer-array run."""
    _bind_stream()
    if not problems:
        return
    L = _lib.lib()
    dt = problems[0].a.data.dtype
    if dt == torch.float32:
        arr = (_lib.BatchProblemF32C * len(problems))(*[
            _lib.BatchProblemF32C(float(p.alpha), p.a._c(dt, "A"), p.b._c(dt, "B"),
                                  float(p.beta), p.c._c(dt, "C")) for p in problems])
        _check(L.gk_gemm_batched_slice_f32(_ws(ws), arr, len(problems), _par(par)))
    elif dt == torch.bfloat16:
        arr = (_lib.BatchProblemBf16C * len(problems))(*[
            _lib.BatchProblemBf16C(_bf16_bits(p.alpha), p.a._c(dt, "A"), p.b._c(dt, "B"),
                                   _bf16_bits(p.beta), p.c._c(dt, "C")) for p in problems])
        _check(L.gk_gemm_batched_slice_bf16(_ws(ws), arr, len(problems), _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_batched_slice supports float32 and bfloat16")


def gemm_batched_unchecked(batch, m, k, n, alpha, a, rsa, csa, a_bs, b, rsb, csb, b_bs, beta,
                           c, rsc, csc, c_bs, par=None, ws=None, a_off=0, b_off=0,
                           c_off=0) -> None:
    """``gemm_batched_unchecked(_with)`` (src/api/batched.rs:594-700).

    ``*_off`` are element offsets of the base pointers (negative strides and
    batch strides walk backwards from there)."""
    _bind_stream()
    L = _lib.lib()
    if a.dtype == torch.float32:
        _check(L.gk_gemm_batched_f32_unchecked(_ws(ws), batch, m, k, n, float(alpha),
                                               _ptr(a, a_off), rsa, csa, a_bs, _ptr(b, b_off),
                                               rsb, csb, b_bs, float(beta), _ptr(c, c_off), rsc,
                                               csc, c_bs, _par(par)))
    elif a.dtype == torch.bfloat16:
        _check(L.gk_gemm_batched_bf16_unchecked(_ws(ws), batch, m, k, n, _bf16_bits(alpha),
                                                _ptr(a, a_off), rsa, csa, a_bs, _ptr(b, b_off),
                                                rsb, csb, b_bs, _bf16_bits(beta),
                                                _ptr(c, c_off), rsc, csc, c_bs, _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_batched_unchecked supports float32 and bfloat16")


def gemm_batched_bf16_f32out(batch: int, alpha: float, a: MatRef, a_batch_stride: int,
                             b: MatRef, b_batch_stride: int, beta: float, c: MatMut,
                             c_batch_stride: int, par: Optional[Parallelism] = None,
                             ws: Optional[Workspace] = None) -> None:
    """Extension: batched bf16 x bf16 -> f32 (attention-score shape)."""
    _bind_stream()
    _check(_lib.lib().gk_gemm_batched_bf16_f32out(
        _ws(ws), batch, float(alpha), a._c(torch.bfloat16, "A"), a_batch_stride,
        b._c(torch.bfloat16, "B"), b_batch_stride, float(beta), c._c(torch.float32, "C"),
        c_batch_stride, _par(par)))


# ------------------------------------------------------ prepacked f32 / bf16 B

def prepack_rhs(b: MatRef) -> PackedRhs:
    """``prepack_rhs::<f32|bf16>`` (src/api/packed.rs:67-170)."""
    _bind_stream()
    L = _lib.lib()
    out = C.c_void_p()
    dt = b.data.dtype
    if dt == torch.float32:
        _check(L.gk_prepack_rhs_f32(b._c(dt, "B"), C.byref(out)))
    elif dt == torch.bfloat16:
        _check(L.gk_prepack_rhs_bf16(b._c(dt, "B"), C.byref(out)))
    else:
        raise TypeError(f"gemmkit_amd: prepack_rhs supports float32 and bfloat16, got {dt}")
    return PackedRhs(out.value)


def gemm_packed_b(alpha, a: MatRef, packed: PackedRhs, beta, c: MatMut,
                  par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_packed_b(_with)`` (src/api/packed.rs:175-260): column-major-ish C."""
    _bind_stream()
    L = _lib.lib()
    dt = a.data.dtype
    if dt == torch.float32:
        _check(L.gk_gemm_packed_b_f32(_ws(ws), float(alpha), a._c(dt, "A"), packed.handle,
                                      float(beta), c._c(dt, "C"), _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_packed_b_bf16(_ws(ws), _bf16_bits(alpha), a._c(dt, "A"), packed.handle,
                                       _bf16_bits(beta), c._c(dt, "C"), _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_packed_b supports float32 and bfloat16, got {dt}")


def gemm_packed_b_unchecked(alpha, m, a, rsa, csa, packed: PackedRhs, beta, c, rsc, csc,
                            par=None, ws=None, a_off=0, c_off=0) -> None:
    """``gemm_packed_b_unchecked(_with)`` (src/api/packed.rs:270-365)."""
    _bind_stream()
    L = _lib.lib()
    if a.dtype == torch.float32:
        _check(L.gk_gemm_packed_b_f32_unchecked(_ws(ws), float(alpha), m, _ptr(a, a_off), rsa, csa,
                                                packed.handle, float(beta), _ptr(c, c_off), rsc,
                                                csc, _par(par)))
    elif a.dtype == torch.bfloat16:
        _check(L.gk_gemm_packed_b_bf16_unchecked(_ws(ws), _bf16_bits(alpha), m, _ptr(a, a_off),
                                                 rsa, csa, packed.handle, _bf16_bits(beta),
                                                 _ptr(c, c_off), rsc, csc, _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_packed_b_unchecked supports float32 and bfloat16")


# ------------------------------------------------------ fused bias/activation

BIAS_PER_ROW = 0
BIAS_PER_COL = 1


class Bias:
    """Bias (src/api/fused.rs:17-23): ``PerRow(tensor)`` (length m) or
    ``PerCol(tensor)`` (length n), of the GEMM's element type."""

    def __init__(self, dim: int, data: torch.Tensor):
        self.dim, self.data = dim, data

    @staticmethod
    def PerRow(data: torch.Tensor) -> "Bias":  # noqa: N802 -- mirrors the Rust variant
        return Bias(BIAS_PER_ROW, data)

    @staticmethod
    def PerCol(data: torch.Tensor) -> "Bias":  # noqa: N802
        return Bias(BIAS_PER_COL, data)

    def _c(self, dtype: torch.dtype) -> BiasC:
        d = _slice(self.data, "bias")
        if d.dtype != dtype:
            raise TypeError(f"gemmkit_amd: bias must be {dtype}, got {d.dtype}")
        return BiasC(d.data_ptr(), d.numel(), self.dim)


class Activation:
    """Activation (src/api/fused.rs:25-31): ``Relu`` or ``LeakyRelu(slope)``."""

    def __init__(self, kind: int, slope: float = 0.0):
        self.kind, self.slope = kind, float(slope)

    @staticmethod
    def LeakyRelu(slope: float) -> "Activation":  # noqa: N802
        return Activation(2, slope)


Activation.Relu = Activation(1)  # type: ignore[attr-defined]


def _fused_args(dt: torch.dtype, bias: Optional[Bias], act: Optional[Activation]):
    """(gk_bias pointer or None, act code, slope in the ABI's scalar type)."""
    bc = None if bias is None else C.byref(bias._c(dt))
    kind = 0 if act is None else act.kind
    slope = 0.0 if act is None else act.slope
    return bc, kind, (_bf16_bits(slope) if dt == torch.bfloat16 else slope)


def _raw_bias(bias: Optional[torch.Tensor], dim: int):
    return _ptr(bias), int(dim), (1 if bias is not None else 0)


def gemm_fused(alpha, a: MatRef, b: MatRef, beta, c: MatMut, bias: Optional[Bias] = None,
               act: Optional[Activation] = None, par: Optional[Parallelism] = None,
               ws: Optional[Workspace] = None) -> None:
    """``gemm_fused(_with)`` (src/api/fused.rs:61-140):
    C <- act(alpha*A*B + beta*C + bias), float32 or bfloat16."""
    _bind_stream()
    L = _lib.lib()
    dt = a.data.dtype
    bc, kind, slope = _fused_args(dt, bias, act)
    if dt == torch.float32:
        _check(L.gk_gemm_fused_f32(_ws(ws), float(alpha), a._c(dt, "A"), b._c(dt, "B"),
                                   float(beta), c._c(dt, "C"), bc, kind, slope, _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_fused_bf16(_ws(ws), _bf16_bits(alpha), a._c(dt, "A"), b._c(dt, "B"),
                                    _bf16_bits(beta), c._c(dt, "C"), bc, kind, slope, _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_fused supports float32 and bfloat16, got {dt}")


def gemm_fused_unchecked(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc,
                         bias=None, bias_dim=BIAS_PER_ROW, act: Optional[Activation] = None,
                         par=None, ws=None, a_off=0, b_off=0, c_off=0) -> None:
    """``gemm_fused_unchecked(_with)`` (src/api/fused.rs:149-230)."""
    _bind_stream()
    L = _lib.lib()
    bp, bd, hb = _raw_bias(bias, bias_dim)
    _, kind, slope = _fused_args(a.dtype, None, act)
    if a.dtype == torch.float32:
        _check(L.gk_gemm_fused_f32_unchecked(_ws(ws), m, k, n, float(alpha), _ptr(a, a_off), rsa,
                                             csa, _ptr(b, b_off), rsb, csb, float(beta),
                                             _ptr(c, c_off), rsc, csc, bp, bd, hb, kind, slope,
                                             _par(par)))
    elif a.dtype == torch.bfloat16:
        _check(L.gk_gemm_fused_bf16_unchecked(_ws(ws), m, k, n, _bf16_bits(alpha), _ptr(a, a_off),
                                              rsa, csa, _ptr(b, b_off), rsb, csb,
                                              _bf16_bits(beta), _ptr(c, c_off), rsc, csc, bp, bd,
                                              hb, kind, slope, _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_fused_unchecked supports float32 and bfloat16")


def gemm_batched_fused(batch: int, alpha, a: MatRef, a_batch_stride: int, b: MatRef,
                       b_batch_stride: int, beta, c: MatMut, c_batch_stride: int,
                       bias: Optional[Bias] = None, act: Optional[Activation] = None,
                       par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_batched_fused(_with)`` (src/api/batched.rs:307-450): one shared bias."""
    _bind_stream()
    L = _lib.lib()
    dt = a.data.dtype
    bc, kind, slope = _fused_args(dt, bias, act)
    if dt == torch.float32:
        _check(L.gk_gemm_batched_fused_f32(_ws(ws), batch, float(alpha), a._c(dt, "A"),
                                           a_batch_stride, b._c(dt, "B"), b_batch_stride,
                                           float(beta), c._c(dt, "C"), c_batch_stride, bc, kind,
                                           slope, _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_batched_fused_bf16(_ws(ws), batch, _bf16_bits(alpha), a._c(dt, "A"),
                                            a_batch_stride, b._c(dt, "B"), b_batch_stride,
                                            _bf16_bits(beta), c._c(dt, "C"), c_batch_stride, bc,
                                            kind, slope, _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_batched_fused supports float32 and bfloat16, got {dt}")


def gemm_batched_fused_unchecked(batch, m, k, n, alpha, a, rsa, csa, a_bs, b, rsb, csb, b_bs,
                                 beta, c, rsc, csc, c_bs, bias=None, bias_dim=BIAS_PER_ROW,
                                 act: Optional[Activation] = None, par=None, ws=None) -> None:
    """``gemm_batched_fused_unchecked(_with)`` (src/api/batched.rs:459-590)."""
    _bind_stream()
    L = _lib.lib()
    bp, bd, hb = _raw_bias(bias, bias_dim)
    _, kind, slope = _fused_args(a.dtype, None, act)
    if a.dtype == torch.float32:
        _check(L.gk_gemm_batched_fused_f32_unchecked(
            _ws(ws), batch, m, k, n, float(alpha), _ptr(a), rsa, csa, a_bs, _ptr(b), rsb, csb,
            b_bs, float(beta), _ptr(c), rsc, csc, c_bs, bp, bd, hb, kind, slope, _par(par)))
    elif a.dtype == torch.bfloat16:
        _check(L.gk_gemm_batched_fused_bf16_unchecked(
            _ws(ws), batch, m, k, n, _bf16_bits(alpha), _ptr(a), rsa, csa, a_bs, _ptr(b), rsb,
            csb, b_bs, _bf16_bits(beta), _ptr(c), rsc, csc, c_bs, bp, bd, hb, kind, slope,
            _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_batched_fused_unchecked supports float32 and bfloat16")


def gemm_packed_b_fused(alpha, a: MatRef, packed: PackedRhs, beta, c: MatMut,
                        bias: Optional[Bias] = None, act: Optional[Activation] = None,
                        par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_packed_b_fused(_with)`` (src/api/packed.rs:684-790)."""
    _bind_stream()
    L = _lib.lib()
    dt = a.data.dtype
    bc, kind, slope = _fused_args(dt, bias, act)
    if dt == torch.float32:
        _check(L.gk_gemm_packed_b_fused_f32(_ws(ws), float(alpha), a._c(dt, "A"), packed.handle,
                                            float(beta), c._c(dt, "C"), bc, kind, slope,
                                            _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_packed_b_fused_bf16(_ws(ws), _bf16_bits(alpha), a._c(dt, "A"),
                                             packed.handle, _bf16_bits(beta), c._c(dt, "C"), bc,
                                             kind, slope, _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_packed_b_fused supports float32 and bfloat16, got {dt}")


def gemm_packed_b_fused_unchecked(alpha, m, a, rsa, csa, packed: PackedRhs, beta, c, rsc, csc,
                                  bias=None, bias_dim=BIAS_PER_ROW,
                                  act: Optional[Activation] = None, par=None, ws=None,
                                  a_off=0, c_off=0) -> None:
    """``gemm_packed_b_fused_unchecked(_with)`` (src/api/packed.rs:801-950)."""
    _bind_stream()
    L = _lib.lib()
    bp, bd, hb = _raw_bias(bias, bias_dim)
    _, kind, slope = _fused_args(a.dtype, None, act)
    if a.dtype == torch.float32:
        _check(L.gk_gemm_packed_b_fused_f32_unchecked(
            _ws(ws), float(alpha), m, _ptr(a, a_off), rsa, csa, packed.handle, float(beta),
            _ptr(c, c_off), rsc, csc, bp, bd, hb, kind, slope, _par(par)))
    elif a.dtype == torch.bfloat16:
        _check(L.gk_gemm_packed_b_fused_bf16_unchecked(
            _ws(ws), _bf16_bits(alpha), m, _ptr(a, a_off), rsa, csa, packed.handle,
            _bf16_bits(beta), _ptr(c, c_off), rsc, csc, bp, bd, hb, kind, slope, _par(par)))
    else:
        raise TypeError("gemmkit_amd: gemm_packed_b_fused_unchecked supports float32 and bfloat16")


# ------------------------------------------------------------ prepacked LHS

class PackedLhs:
    """PackedLhs<T> (src/api/packed.rs:953-981): A packed once on the device,
    float32 or bfloat16 (:func:`prepack_lhs`)."""

    def __init__(self, handle, dtype: torch.dtype):
        self._free = _lib.lib().gk_packed_lhs_free  # held so __del__ works during interpreter exit
        self._h = handle
        self.dtype = dtype

    @property
    def handle(self):
        return self._h

    def rows(self) -> int:
        return int(_lib.lib().gk_packed_lhs_rows(self._h))

    def cols(self) -> int:
        return int(_lib.lib().gk_packed_lhs_cols(self._h))

    def __del__(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._free(h)


def prepack_lhs(a: MatRef) -> PackedLhs:
    """``prepack_lhs::<f32|bf16>`` (src/api/packed.rs:986-996)."""
    _bind_stream()
    L = _lib.lib()
    out = C.c_void_p()
    dt = a.data.dtype
    if dt == torch.float32:
        _check(L.gk_prepack_lhs_f32(a._c(dt, "A"), C.byref(out)))
    elif dt == torch.bfloat16:
        _check(L.gk_prepack_lhs_bf16(a._c(dt, "A"), C.byref(out)))
    else:
        raise TypeError(f"gemmkit_amd: prepack_lhs supports float32 and bfloat16, got {dt}")
    return PackedLhs(out.value, dt)


def prepack_lhs_unchecked(a: torch.Tensor, rsa, csa, m, k, a_off=0) -> PackedLhs:
    """``prepack_lhs_unchecked`` (src/api/packed.rs:999-1030)."""
    _bind_stream()
    L = _lib.lib()
    out = C.c_void_p()
    fn = L.gk_prepack_lhs_f32_unchecked if a.dtype == torch.float32 else \
        L.gk_prepack_lhs_bf16_unchecked
    _check(fn(_ptr(a, a_off), rsa, csa, m, k, C.byref(out)))
    return PackedLhs(out.value, a.dtype)


def gemm_packed_a(alpha, packed: PackedLhs, b: MatRef, beta, c: MatMut,
                  par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_packed_a(_with)`` (src/api/packed.rs:1049-1140): row-major-ish C."""
    _bind_stream()
    L = _lib.lib()
    dt = b.data.dtype
    if dt == torch.float32:
        _check(L.gk_gemm_packed_a_f32(_ws(ws), float(alpha), packed.handle, b._c(dt, "B"),
                                      float(beta), c._c(dt, "C"), _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_packed_a_bf16(_ws(ws), _bf16_bits(alpha), packed.handle, b._c(dt, "B"),
                                       _bf16_bits(beta), c._c(dt, "C"), _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_packed_a supports float32 and bfloat16, got {dt}")


def gemm_packed_a_unchecked(alpha, packed: PackedLhs, n, b, rsb, csb, beta, c, rsc, csc,
                            par=None, ws=None, b_off=0, c_off=0) -> None:
    """``gemm_packed_a_unchecked(_with)`` (src/api/packed.rs:1143-1240)."""
    _bind_stream()
    L = _lib.lib()
    if b.dtype == torch.float32:
        _check(L.gk_gemm_packed_a_f32_unchecked(_ws(ws), float(alpha), packed.handle, n,
                                                _ptr(b, b_off), rsb, csb, float(beta),
                                                _ptr(c, c_off), rsc, csc, _par(par)))
    else:
        _check(L.gk_gemm_packed_a_bf16_unchecked(_ws(ws), _bf16_bits(alpha), packed.handle, n,
                                                 _ptr(b, b_off), rsb, csb, _bf16_bits(beta),
                                                 _ptr(c, c_off), rsc, csc, _par(par)))


def gemm_packed_a_fused(alpha, packed: PackedLhs, b: MatRef, beta, c: MatMut,
                        bias: Optional[Bias] = None, act: Optional[Activation] = None,
                        par: Optional[Parallelism] = None, ws: Optional[Workspace] = None) -> None:
    """``gemm_packed_a_fused(_with)`` (src/api/packed.rs:1250-1365)."""
    _bind_stream()
    L = _lib.lib()
    dt = b.data.dtype
    bc, kind, slope = _fused_args(dt, bias, act)
    if dt == torch.float32:
        _check(L.gk_gemm_packed_a_fused_f32(_ws(ws), float(alpha), packed.handle, b._c(dt, "B"),
                                            float(beta), c._c(dt, "C"), bc, kind, slope,
                                            _par(par)))
    elif dt == torch.bfloat16:
        _check(L.gk_gemm_packed_a_fused_bf16(_ws(ws), _bf16_bits(alpha), packed.handle,
                                             b._c(dt, "B"), _bf16_bits(beta), c._c(dt, "C"), bc,
                                             kind, slope, _par(par)))
    else:
        raise TypeError(f"gemmkit_amd: gemm_packed_a_fused supports float32 and bfloat16, got {dt}")


def gemm_packed_a_fused_unchecked(alpha, packed: PackedLhs, n, b, rsb, csb, beta, c, rsc, csc,
                                  bias=None, bias_dim=0, act=0, slope=0.0, par=None, ws=None,
                                  b_off=0, c_off=0) -> None:
    """``gemm_packed_a_fused_unchecked(_with)`` (src/api/packed.rs:1369-1440)."""
    _bind_stream()
    L = _lib.lib()
    bp, bd, hb = _raw_bias(bias, bias_dim)
    if b.dtype == torch.float32:
        _check(L.gk_gemm_packed_a_fused_f32_unchecked(
            _ws(ws), float(alpha), packed.handle, n, _ptr(b, b_off), rsb, csb, float(beta),
            _ptr(c, c_off), rsc, csc, bp, bd, hb, int(act), float(slope), _par(par)))
    else:
        _check(L.gk_gemm_packed_a_fused_bf16_unchecked(
            _ws(ws), _bf16_bits(alpha), packed.handle, n, _ptr(b, b_off), rsb, csb,
            _bf16_bits(beta), _ptr(c, c_off), rsc, csc, bp, bd, hb, int(act), _bf16_bits(slope),
            _par(par)))
