"""Test helpers: build strided operands on the host and mirror them on the device."""
from __future__ import annotations

import numpy as np
import torch


def layout_strides(rows: int, cols: int, layout: str, pad: int = 0):
    """(rs, cs, buffer length) of a rows x cols view: 'row', 'col', or a padded
    'row+'/'col+' variant with `pad` extra elements per leading dimension."""
    if layout == "row":
        return cols, 1, rows * cols
    if layout == "col":
        return 1, rows, rows * cols
    if layout == "row+":
        ld = cols + pad
        return ld, 1, rows * ld
    if layout == "col+":
        ld = rows + pad
        return 1, ld, cols * ld
    raise ValueError(layout)


def scatter(dense: np.ndarray, rs: int, cs: int, length: int, fill=0) -> np.ndarray:
    """Place a dense row-major matrix into a flat buffer at strides (rs, cs)."""
    rows, cols = dense.shape
    buf = np.full(length, fill, dtype=dense.dtype)
    ii, jj = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    buf[(ii * rs + jj * cs).ravel()] = dense.ravel()
    return buf


def gather(buf: np.ndarray, rows: int, cols: int, rs: int, cs: int, off: int = 0) -> np.ndarray:
    ii, jj = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    return buf[(off + ii * rs + jj * cs).ravel()].reshape(rows, cols)


def to_dev(x: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def bf16_tensor_from_bits(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).to(dev).view(torch.bfloat16)


def rel_errors(got: np.ndarray, ref: np.ndarray, floor_frac: float = 1e-3):
    """(floored, unfloored) maximum relative error of got against ref: the
    floored one divides by max(|ref|, floor_frac * max|ref|), the unfloored one
    by |ref| over the elements where ref != 0."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    err = np.abs(got - ref)
    floor = floor_frac * np.abs(ref).max()
    floored = float((err / np.maximum(np.abs(ref), floor)).max())
    nz = ref != 0
    unfloored = float((err[nz] / np.abs(ref[nz])).max()) if nz.any() else 0.0
    return floored, unfloored
