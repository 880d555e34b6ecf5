"""CPU-side checks of the C-ABI library: it loads, exports every entry point the
header declares, and its pure host functions (geometry, argument validation)
behave as documented. No GPU work is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmm_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from inference_amd import qmm
    return qmm.lib()


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("qmm_qtensor_from_ggml", "qmm_qtensor_quantize", "qmm_matmul", "qmm_quantize_rows",
                 "qmm_block_dots", "qmm_qtensor_dequantize"):
        assert must in names


def test_library_exports_every_declared_symbol(L):
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, f"libqmm.so lacks {missing}"


def test_python_binding_covers_the_header():
    from inference_amd import qmm
    assert sorted(qmm.EXPORTS) == declared_functions()


def _c_params():
    """{function: [parameter names]} of the header's declarations."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(qmm_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = " ".join(args.split())
        out[name] = [] if args in ("", "void") else [re.search(r"(\w+)$", a.strip()).group(1)
                                                    for a in args.split(",")]
    return out


def test_rust_sys_bindings_mirror_the_header():
    """include/qmm_sys.rs (the Rust -sys layer; no Rust toolchain here) declares every header function
    with the same parameter names in the same order (a Rust keyword gets a trailing underscore)."""
    rs = open(os.path.join(ROOT, "include", "qmm_sys.rs")).read()
    block = rs[rs.index('extern "C" {'):rs.index("\n}\n", rs.index('extern "C" {'))]
    rust = {}
    for name, args in re.findall(r"pub fn (qmm_[a-z0-9_]+)\(([^)]*)\)", block, flags=re.S):
        rust[name] = [a.split(":")[0].strip().rstrip("_") for a in " ".join(args.split()).split(",") if a.strip()]
    c = _c_params()
    assert sorted(rust) == sorted(c) == declared_functions()
    for name, params in c.items():
        assert rust[name] == params, name


def test_rust_from_ggml_checks_the_slice_length():
    """The safe Rust wrapper over qmm_qtensor_from_ggml (which copies n * (k / block) * type_size bytes from
    the host pointer) refuses a slice of any other length before the call: a safe call cannot read past it.
    No Rust toolchain here, so the order is checked in the source: the length comparison, with checked
    arithmetic, precedes the only unsafe call of the function."""
    rs = open(os.path.join(ROOT, "include", "qmm_sys.rs")).read()
    body = rs[rs.index("pub fn from_ggml("):]
    body = body[:body.index("\n    }\n")]
    call = body.index("qmm_qtensor_from_ggml(")
    assert "bytes.len()" in body[:call] and "checked_mul" in body[:call]
    assert body.index("return Err(invalid(\"byte slice length") < call


def test_geometry(L):
    # crates/llm/mlx-llm/src/gguf/dequant.rs:752-773 (block geometry KAT)
    assert (L.qmm_block_size(8), L.qmm_type_size(8)) == (32, 34)
    assert (L.qmm_block_size(12), L.qmm_type_size(12)) == (256, 144)
    assert (L.qmm_block_size(14), L.qmm_type_size(14)) == (256, 210)
    assert (L.qmm_block_size(15), L.qmm_type_size(15)) == (256, 292)
    assert L.qmm_vec_dot_type(8) == 8 and L.qmm_vec_dot_type(12) == 15 and L.qmm_vec_dot_type(14) == 15
    assert L.qmm_block_size(3) == -1 and L.qmm_vec_dot_type(15) == -1


def test_argument_errors_before_any_gpu_call(L):
    """Shape/dtype validation happens on the host and reports QMM_ERR_INVALID."""
    h = ctypes.c_void_p()
    buf = (ctypes.c_uint8 * 144)()
    # k not a multiple of 256 (prepare.rs:236-243 rejects such shapes too)
    rc = L.qmm_qtensor_from_ggml(12, 1, 200, buf, 0, None, ctypes.byref(h))
    assert rc == 1 and b"multiple" in L.qmm_last_error()
    rc = L.qmm_qtensor_from_ggml(15, 1, 256, buf, 0, None, ctypes.byref(h))  # Q8K is activation-only
    assert rc == 1
    rc = L.qmm_qtensor_from_ggml(12, 1, 256, None, 0, None, ctypes.byref(h))
    assert rc == 1
    x = (ctypes.c_float * 256)()
    assert L.qmm_quantize_rows(12, x, 1, 256, 256, buf, None) == 1  # not a vec-dot type
    assert L.qmm_quantize_rows(15, x, 1, 100, 100, buf, None) == 1  # k % 256
    assert L.qmm_quantize_rows(15, x, 1, 256, 128, buf, None) == 1  # ldx < k
    assert L.qmm_matmul_workspace_size(None, 1) == 0
    assert L.qmm_qtensor_ggml_bytes(None) == 0
    L.qmm_qtensor_free(None)


def test_python_api_validates_on_host():
    from inference_amd import GgmlDType, QmmError, QuantSpec
    assert QuantSpec.q4().dtype == GgmlDType.Q4K and QuantSpec.q8().dtype == GgmlDType.Q8_0
    assert QuantSpec.from_bits(4) == QuantSpec.q4() and QuantSpec.from_bits(8) == QuantSpec.q8()
    assert QuantSpec.from_bits(6) is None
    assert QuantSpec.q4().bits() == 4 and QuantSpec.q8().bits() == 8
    assert GgmlDType.Q4K.vec_dot_type() == GgmlDType.Q8K
    import torch
    with pytest.raises(QmmError):
        from inference_amd import quantize_rows
        quantize_rows(GgmlDType.Q8K, torch.zeros(1, 256))  # CPU tensor: rejected, no fallback


def test_quantize_onto_source_rules():
    """QTensor::quantize_onto takes a host, contiguous, zero-offset source (candle-gen/src/quant/mod.rs:693-717)
    and a GPU target; everything else is rejected before any device work."""
    import torch
    from inference_amd import GgmlDType, QmmError, QTensor
    w = torch.zeros(8, 512)
    with pytest.raises(QmmError, match="contiguous"):
        QTensor.quantize_onto(w.t(), GgmlDType.Q4K, torch.device("cuda:0"))
    with pytest.raises(QmmError, match="contiguous"):
        QTensor.quantize_onto(w[1:], GgmlDType.Q4K, torch.device("cuda:0"))  # nonzero offset
    with pytest.raises(QmmError, match="GPU"):
        QTensor.quantize_onto(w, GgmlDType.Q4K, torch.device("cpu"))
