"""CPU tests of the C ABI: the library loads without a GPU, exports every
symbol include/gemmkit_hip.h declares, and the checked tier rejects invalid
views with the reference's exact panic messages (src/api.rs:188-314,
src/adapter.rs:130-273, src/api/int8.rs:291-295, src/api/batched.rs:31-163)
before touching the device.  No compute entry point runs here."""
import ctypes as C
import os
import re

import pytest

from gemmkit_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gemmkit_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for must in ("gk_gemm_f32", "gk_gemm_bf16", "gk_gemm_bf16_f32out", "gk_gemm_i8",
                 "gk_gemm_i8_requant", "gk_gemm_i8_requant_u8", "gk_prepack_rhs_i8",
                 "gk_gemm_i8_packed_b", "gk_packed_rhs_free", "gk_gemm_batched_f32",
                 "gk_gemm_batched_bf16_f32out", "gk_gemm_i8_unchecked"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 36
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


FAKE_A, FAKE_B, FAKE_C = 0x10000, 0x20000, 0x30000


def ref(data, length, rows, cols, rs, cs):
    return _lib.MatRefC(data, length, rows, cols, rs, cs)


def mut(data, length, rows, cols, rs, cs):
    return _lib.MatMutC(data, length, rows, cols, rs, cs)


def call_i8(a, b, c):
    L = _lib.lib()
    rc = L.gk_gemm_i8(None, 1, C.byref(a), C.byref(b), 0, C.byref(c), 1)
    return rc, _lib.last_error()


@pytest.mark.parametrize("a,b,c,code,msg", [
    (ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 9, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1),
     -1, "gemmkit: A.cols (10) != B.rows (9)"),
    (ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 9, 10, 10, 1),
     -1, "gemmkit: A.rows (10) != C.rows (9)"),
    (ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 9, 9, 1), mut(FAKE_C, 100, 10, 10, 10, 1),
     -1, "gemmkit: B.cols (9) != C.cols (10)"),
    (ref(FAKE_A, 99, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1),
     -2, "gemmkit: A view of 10x10 (strides 10,1) needs 100 elements but slice has 99"),
    (ref(FAKE_A, 100, 10, 10, -10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1),
     -2, "gemmkit: A view has negative strides or is too large to address; use gemm_unchecked"),
    (ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 0, 1),
     -3, "gemmkit: C view aliases itself (strides 0,1 map distinct elements to the same memory); "
         "C must address each (i,j) uniquely"),
    (ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 5, 1),
     -3, "gemmkit: C view aliases itself (strides 5,1 map distinct elements to the same memory); "
         "C must address each (i,j) uniquely"),
    (ref(FAKE_C + 200, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1),
     -3, "gemmkit: C aliases A or B"),
])
def test_checked_gemm_i8_validation(a, b, c, code, msg):
    rc, err = call_i8(a, b, c)
    assert rc == code
    assert err == msg


def requant(scale=0.5, zp=0, scales=None, scales_len=0, bias=None, bias_len=0, axis=0, act=0):
    return _lib.RequantizeC(scale, scales, scales_len, zp, bias, bias_len, axis, act)


@pytest.mark.parametrize("req,u8,msg", [
    (requant(scale=0.0), False, "gemmkit: requantize scale (0) must be finite and > 0"),
    (requant(scale=-1.5), False, "gemmkit: requantize scale (-1.5) must be finite and > 0"),
    (requant(scale=float("nan")), False, "gemmkit: requantize scale (NaN) must be finite and > 0"),
    (requant(scale=float("inf")), False, "gemmkit: requantize scale (inf) must be finite and > 0"),
    (requant(zp=128), False, "gemmkit: requantize zero_point (128) out of i8 range [-128, 127]"),
    (requant(zp=-129), False, "gemmkit: requantize zero_point (-129) out of i8 range [-128, 127]"),
    (requant(zp=-1), True, "gemmkit: requantize zero_point (-1) out of u8 range [0, 255]"),
    (requant(zp=256), True, "gemmkit: requantize zero_point (256) out of u8 range [0, 255]"),
    (requant(bias=0x50000, bias_len=3), False, "gemmkit: requantize bias length (3) != A.rows (10)"),
    (requant(bias=FAKE_C + 4, bias_len=10), False, "gemmkit: requantize bias overlaps C"),
    (requant(scales=0x60000, scales_len=4), False,
     "gemmkit: requantize scales length (4) != A.rows (10)"),
    (requant(scales=FAKE_C, scales_len=10), False, "gemmkit: requantize scales overlap C"),
    (requant(bias=0x50000, bias_len=10, axis=1), False,
     "gemmkit: requantize bias length (10) != B.cols (12)"),
])
def test_checked_requant_validation(req, u8, msg):
    L = _lib.lib()
    a = ref(FAKE_A, 100, 10, 10, 10, 1)
    b = ref(FAKE_B, 120, 10, 12, 12, 1)
    c = mut(FAKE_C, 120, 10, 12, 12, 1)
    fn = L.gk_gemm_i8_requant_u8 if u8 else L.gk_gemm_i8_requant
    rc = fn(None, C.byref(a), C.byref(b), C.byref(req), C.byref(c), 1)
    assert rc < 0
    assert _lib.last_error() == msg


def test_rust_float_formatting_of_scale():
    L = _lib.lib()
    a = ref(FAKE_A, 100, 10, 10, 10, 1)
    b = ref(FAKE_B, 120, 10, 12, 12, 1)
    c = mut(FAKE_C, 120, 10, 12, 12, 1)
    for s, text in ((-1e30, "-1000000000000000000000000000000"), (-1e-9, "-0.000000001"),
                    (-0.1, "-0.1"), (-3.0, "-3"), (-0.0, "-0")):
        r = requant(scale=s)
        assert L.gk_gemm_i8_requant(None, C.byref(a), C.byref(b), C.byref(r), C.byref(c), 1) < 0
        assert _lib.last_error() == f"gemmkit: requantize scale ({text}) must be finite and > 0"


@pytest.mark.parametrize("batch,a_bs,c_bs,c,msg", [
    (3, -1, 100, mut(FAKE_C, 1000, 10, 10, 10, 1),
     "gemmkit: A batch stride (-1) must be non-negative"),
    (3, 100, 100, mut(FAKE_C, 250, 10, 10, 10, 1),
     "gemmkit: C batched view (3× 10x10, batch stride 100) needs 300 elements but slice has 250"),
    (3, 100, 50, mut(FAKE_C, 1000, 10, 10, 10, 1),
     "gemmkit: C batch stride (50) must be at least the element extent (100) so the batched C "
     "outputs stay disjoint"),
    (3, 100, 100, mut(FAKE_C, 1000, 10, 10, 10, -1),
     "gemmkit: C view has negative strides or is too large to address; use the unchecked API"),
])
def test_checked_batched_validation(batch, a_bs, c_bs, c, msg):
    L = _lib.lib()
    a = ref(FAKE_A, 1000, 10, 10, 10, 1)
    b = ref(FAKE_B, 1000, 10, 10, 10, 1)
    rc = L.gk_gemm_batched_f32(None, batch, 1.0, C.byref(a), a_bs, C.byref(b), 100, 0.0,
                               C.byref(c), c_bs, 1)
    assert rc < 0
    assert _lib.last_error() == msg


def test_packed_b_layout_rule_message():
    # gemm_i8_packed_b_unchecked asserts a column-major-ish C before anything
    # else (src/api/packed.rs:625-629); a null handle reports first here, so use
    # the checked shape path with a fake handle only for the layout message.
    L = _lib.lib()
    rc = L.gk_gemm_i8_packed_b_unchecked(None, 1, 4, FAKE_A, 8, 1, None, 0, FAKE_C, 8, 1, 1)
    assert rc < 0 and _lib.last_error() == "gemmkit: null packed RHS"


def test_python_mirror_raises_reference_message():
    import torch
    import gemmkit_amd as gk
    a = torch.zeros(10)
    with pytest.raises(gk.GemmkitError) as e:
        gk.gemm(1.0, gk.MatRef(a, 2, 5, 5, 1), gk.MatRef(a, 4, 2, 2, 1), 0.0, gk.MatMut(a, 2, 2, 2, 1))
    assert "HIP device" in str(e.value)


def bias(data, length, dim):
    return _lib.BiasC(data, length, dim)


# Fused-entry checks (src/api/fused.rs:81-110, src/adapter.rs:130-166; the
# reference's own cases are tests/epilogue/float.rs:400-470).
@pytest.mark.parametrize("bs,act,slope,code,msg", [
    (bias(0x50000, 3, 0), 0, 0.0, -1, "gemmkit: PerRow bias length (3) != A.rows (4)"),
    (bias(0x50000, 4, 1), 0, 0.0, -1, "gemmkit: PerCol bias length (4) != B.cols (6)"),
    (None, 2, float("inf"), -4, "gemmkit: LeakyRelu slope must be finite"),
    (None, 2, float("nan"), -4, "gemmkit: LeakyRelu slope must be finite"),
    (bias(FAKE_C, 4, 0), 0, 0.0, -3, "gemmkit: bias slice overlaps C"),
    (bias(FAKE_C + 2 * 23, 6, 1), 1, 0.0, -3, "gemmkit: bias slice overlaps C"),
    (bias(0x50000, 4, 7), 0, 0.0, -4, "gemmkit: bias dim (7) must be 0 (PerRow) or 1 (PerCol)"),
    (None, 3, 0.0, -4, "gemmkit: activation (3) must be 0 (none), 1 (Relu) or 2 (LeakyRelu)"),
])
def test_checked_fused_validation(bs, act, slope, code, msg):
    L = _lib.lib()
    a = ref(FAKE_A, 16, 4, 4, 4, 1)
    b = ref(FAKE_B, 24, 4, 6, 6, 1)
    c = mut(FAKE_C, 24, 4, 6, 6, 1)
    bp = C.byref(bs) if bs is not None else None
    rc = L.gk_gemm_fused_f32(None, 1.0, C.byref(a), C.byref(b), 0.0, C.byref(c), bp, act, slope, 1)
    assert (rc, _lib.last_error()) == (code, msg)
    # The bf16 entry checks the same conditions (bias and C in 2-byte elements:
    # the overlap cases keep overlapping).
    slope_bits = 0x7F80 if slope == float("inf") else (0x7FC0 if slope != slope else 0)
    rc = L.gk_gemm_fused_bf16(None, 0x3F80, C.byref(a), C.byref(b), 0, C.byref(c), bp, act,
                              slope_bits, 1)
    assert (rc, _lib.last_error()) == (code, msg)


def test_checked_fused_view_checks_come_first():
    # validate_gemm_views runs before the bias checks (src/api/fused.rs:98-101).
    L = _lib.lib()
    a = ref(FAKE_A, 16, 4, 4, 4, 1)
    b = ref(FAKE_B, 24, 3, 6, 6, 1)
    c = mut(FAKE_C, 24, 4, 6, 6, 1)
    bs = bias(0x50000, 3, 0)
    rc = L.gk_gemm_fused_f32(None, 1.0, C.byref(a), C.byref(b), 0.0, C.byref(c), C.byref(bs),
                             0, 0.0, 1)
    assert rc == -1 and _lib.last_error() == "gemmkit: A.cols (4) != B.rows (3)"


def test_checked_batched_fused_validation():
    L = _lib.lib()
    a = ref(FAKE_A, 1000, 10, 10, 10, 1)
    b = ref(FAKE_B, 1000, 10, 10, 10, 1)
    c = mut(FAKE_C, 1000, 10, 10, 10, 1)
    # The bias is one shared vector sized for a single element.
    bs = bias(0x90000, 30, 0)
    rc = L.gk_gemm_batched_fused_f32(None, 3, 1.0, C.byref(a), 100, C.byref(b), 100, 0.0,
                                     C.byref(c), 100, C.byref(bs), 0, 0.0, 1)
    assert rc == -1 and _lib.last_error() == "gemmkit: PerRow bias length (30) != A.rows (10)"
    bs = bias(FAKE_C + 4 * 999, 10, 1)
    rc = L.gk_gemm_batched_fused_f32(None, 3, 1.0, C.byref(a), 100, C.byref(b), 100, 0.0,
                                     C.byref(c), 100, C.byref(bs), 0, 0.0, 1)
    assert rc == -3 and _lib.last_error() == "gemmkit: bias slice overlaps C"
    # batch == 0 returns before any check.
    rc = L.gk_gemm_batched_fused_f32(None, 0, 1.0, C.byref(a), -5, C.byref(b), 100, 0.0,
                                     C.byref(c), 100, C.byref(bs), 0, 0.0, 1)
    assert rc == 0


def test_packed_fused_null_handle():
    L = _lib.lib()
    a = ref(FAKE_A, 16, 4, 4, 4, 1)
    c = mut(FAKE_C, 24, 4, 6, 1, 4)
    rc = L.gk_gemm_packed_b_fused_f32(None, 1.0, C.byref(a), None, 0.0, C.byref(c), None, 1,
                                      0.0, 1)
    assert rc == -4 and _lib.last_error() == "gemmkit: null argument"
    rc = L.gk_gemm_packed_b_f32_unchecked(None, 1.0, 4, FAKE_A, 4, 1, None, 0.0, FAKE_C, 1, 4, 1)
    assert rc == -4 and _lib.last_error() == "gemmkit: null packed RHS"


def batch_problem(a, b, c, alpha=1.0, beta=0.0):
    return _lib.BatchProblemF32C(alpha, a, b, beta, c)


@pytest.mark.parametrize("bad,msg", [
    ((ref(FAKE_A, 100, 10, 9, 9, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1)),
     "gemmkit: batch element 1 A.cols (9) != B.rows (10)"),
    ((ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 9, 10, 10, 1)),
     "gemmkit: batch element 1 A.rows (10) != C.rows (9)"),
    ((ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 9, 9, 1), mut(FAKE_C, 100, 10, 10, 10, 1)),
     "gemmkit: batch element 1 B.cols (9) != C.cols (10)"),
    ((ref(FAKE_A, 99, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1)),
     "gemmkit: A view of 10x10 (strides 10,1) needs 100 elements but slice has 99"),
    ((ref(FAKE_A, 100, 10, 10, -10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 10, 1)),
     "gemmkit: A view has negative strides or is too large to address; use gemm_unchecked"),
    ((ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1), mut(FAKE_C, 100, 10, 10, 5, 1)),
     "gemmkit: batch element 1 C view aliases itself (strides 5,1); C must address each (i,j) "
     "uniquely"),
])
def test_batched_slice_validation(bad, msg):
    # element 0 is valid; element 1 fails with gemm_batched_slice's message
    # (src/api/batched.rs:751-783), before any device work
    ok = batch_problem(ref(FAKE_A, 100, 10, 10, 10, 1), ref(FAKE_B, 100, 10, 10, 10, 1),
                       mut(FAKE_C + 4096, 100, 10, 10, 10, 1))
    arr = (_lib.BatchProblemF32C * 2)(ok, batch_problem(*bad))
    rc = _lib.lib().gk_gemm_batched_slice_f32(None, arr, 2, 1)
    assert rc < 0
    assert _lib.last_error() == msg


def test_batched_ptr_empty_is_a_no_op():
    assert _lib.lib().gk_gemm_batched_ptr_f32_unchecked(None, None, 0, 1) == 0
    assert _lib.lib().gk_gemm_batched_slice_bf16(None, None, 0, 1) == 0
