"""C-ABI checks that need no GPU: both libraries load, export every function
declared in include/*.h, and their pure host helpers (layout constants,
dispatch predicates, layer-kind tables) agree with the reference/oracle."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import edgexpu_amd as E
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header: str) -> list[str]:
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(edgexpu_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


@pytest.mark.parametrize("header,lib", [("edgexpu_hip.h", E.HIP_SO), ("edgexpu_kernels.h", E.KERNELS_SO),
                                        ("edgexpu_gguf_upload.h", E.KERNELS_SO)])
def test_every_declared_symbol_is_exported(header, lib):
    assert os.path.exists(lib), f"{lib} not built"
    names = declared(header)
    assert len(names) >= 8
    handle = C.CDLL(lib)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, f"{os.path.basename(lib)} lacks {missing}"


def test_reference_entry_points_present():
    """The drop-in set carries the reference's own names (cpu_kernel.h / gguf_quant.h)."""
    ref_names = ["edgexpu_cpu_linear_quant", "edgexpu_cpu_linear_quant_batch", "edgexpu_gguf_dequantize",
                 "edgexpu_gguf_quantize_q8_0", "edgexpu_gguf_quantize_q8_k", "edgexpu_gguf_dot_quant",
                 "edgexpu_gguf_dot_quant_q8", "edgexpu_gguf_dot_quant_q8k", "edgexpu_gguf_row_bytes",
                 "edgexpu_gguf_type_block_size", "edgexpu_gguf_type_block_bytes", "edgexpu_gguf_q8_0_nbytes",
                 "edgexpu_gguf_q8_k_nbytes", "edgexpu_gguf_can_dot_q8", "edgexpu_gguf_can_dot_q8k",
                 "edgexpu_gguf_dequantize_row", "edgexpu_gguf_dequantize_q8_0_rows", "edgexpu_gguf_q8_0_dot_row",
                 "edgexpu_gguf_tensor_elements", "edgexpu_gguf_tensor_nbytes", "edgexpu_gguf_quant_selftest",
                 "edgexpu_cpu_softmax", "edgexpu_cpu_sample_softmax"]
    lib = C.CDLL(E.KERNELS_SO)
    assert all(hasattr(lib, n) for n in ref_names)


def test_layout_helpers_match_oracle(ora):
    k = C.CDLL(E.KERNELS_SO)
    for f in ("edgexpu_gguf_type_block_size", "edgexpu_gguf_type_block_bytes"):
        getattr(k, f).restype = C.c_size_t
    k.edgexpu_gguf_row_bytes.restype = C.c_size_t
    k.edgexpu_gguf_q8_0_nbytes.restype = C.c_size_t
    k.edgexpu_gguf_q8_k_nbytes.restype = C.c_size_t
    bs = ora.fn("ora_block_size", C.c_size_t, [C.c_uint32])
    bb = ora.fn("ora_block_bytes", C.c_size_t, [C.c_uint32])
    rb = ora.fn("ora_row_bytes", C.c_size_t, [C.c_uint32, C.c_int])
    for t in list(range(16)) + [99]:
        assert k.edgexpu_gguf_type_block_size(t) == bs(t)
        assert k.edgexpu_gguf_type_block_bytes(t) == bb(t)
        for n in (0, -32, 31, 32, 256, 576, 4096, 14336):
            assert k.edgexpu_gguf_row_bytes(t, n) == rb(t, n)
    for n in (0, 31, 32, 576, 4096):
        assert k.edgexpu_gguf_q8_0_nbytes(n) == (0 if n <= 0 or n % 32 else n // 32 * 34)
        assert k.edgexpu_gguf_q8_k_nbytes(n) == (0 if n <= 0 or n % 256 else n // 256 * 292)
    # dispatch predicates, src/gguf_dot_q8.c:414-434
    assert [t for t in range(16) if k.edgexpu_gguf_can_dot_q8(t)] == [2, 6, 8]
    assert [t for t in range(16) if k.edgexpu_gguf_can_dot_q8k(t)] == [12, 13, 14]


def test_hip_host_helpers_without_gpu():
    L = E.HipLib()
    # every type of the reference's dispatcher (src/gguf_quant.c:69-108)
    assert [t for t in range(16) if L.supports_type(t)] == [0, 1, 2, 6, 8, 12, 13, 14]
    assert L.row_bytes(12, 4096) == 2304 and L.row_bytes(14, 9728) == 7980 and L.row_bytes(8, 576) == 612
    assert L.row_bytes(2, 576) == 324 and L.row_bytes(6, 1536) == 1056 and L.row_bytes(13, 2560) == 1760
    assert L.row_bytes(1, 576) == 1152 and L.row_bytes(1, 7) == 14
    assert L.row_bytes(0, 64) == 256 and L.row_bytes(0, 7) == 28
    assert L.row_bytes(12, 100) == 0 and L.row_bytes(2, 48) == 0 and L.row_bytes(5, 64) == 0


def test_layer_kind_projection_tables():
    k = C.CDLL(E.KERNELS_SO)
    buf = (C.c_int * 16)()
    # EDGEXPU_LAYER_ATTN_SWIGLU: q k v o gate up down (src/native.c:2530-2580)
    assert k.edgexpu_kernels_layer_projections(0, buf, 16) == 7
    assert list(buf[:7]) == [0, 1, 2, 3, 4, 5, 6]
    assert k.edgexpu_kernels_layer_projections(1, buf, 16) == 0        # UNSUPPORTED
    assert k.edgexpu_kernels_layer_projections(2, buf, 16) == 8        # GATED_DELTA
    assert list(buf[:8]) == [7, 8, 9, 10, 11, 4, 5, 6]
    assert k.edgexpu_kernels_layer_projections(3, buf, 16) == 7        # ATTN_QK_NORM
    assert k.edgexpu_kernels_layer_projections(0, None, 0) == 7        # size query


def test_kernel_set_table():
    k = C.CDLL(E.KERNELS_SO)

    class KS(C.Structure):
        _fields_ = [("name", C.c_char_p)] + [(f, C.c_void_p) for f in (
            "linear_quant", "linear_quant_batch", "dequantize", "quantize_q8_0", "quantize_q8_k",
            "dot_quant", "dot_quant_q8", "dot_quant_q8k")]

    k.edgexpu_kernels_hip.restype = C.POINTER(KS)
    ks = k.edgexpu_kernels_hip().contents
    assert ks.name == b"hip.gfx950"
    assert C.cast(k.edgexpu_cpu_linear_quant_batch, C.c_void_p).value == ks.linear_quant_batch
    assert all(getattr(ks, f) for f, _ in KS._fields_[1:])


class _Tensor(C.Structure):
    """include/edgexpu/gguf.h:21-27 layout."""
    _fields_ = [("name", C.c_char * 96), ("n_dims", C.c_uint32), ("type", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_uint64)]


def _tensor(qtype, dims):
    t = _Tensor()
    t.n_dims = len(dims)
    t.type = qtype
    for i, d in enumerate(dims):
        t.dims[i] = d
    return t


def test_tensor_sizes_and_row_checks_without_gpu():
    """edgexpu_gguf_tensor_elements / _nbytes (src/gguf_quant.c:110-136) and the
    argument checks of edgexpu_gguf_dequantize_row (:442-463), which fail
    before any GPU work with the reference's messages."""
    k = C.CDLL(E.KERNELS_SO)
    k.edgexpu_gguf_tensor_elements.restype = C.c_uint64
    k.edgexpu_gguf_tensor_nbytes.restype = C.c_size_t
    for qtype, dims, nbytes in ((12, (4096, 32000), 32000 * 2304), (8, (576, 49152), 49152 * 612),
                                (1, (7, 3), 42), (13, (2560, 10), 17600), (12, (100, 3), 0), (5, (64,), 0)):
        t = _tensor(qtype, dims)
        assert k.edgexpu_gguf_tensor_elements(C.byref(t)) == int(np.prod(dims))
        assert k.edgexpu_gguf_tensor_nbytes(C.byref(t)) == nbytes
    assert k.edgexpu_gguf_tensor_nbytes(None) == 0 and k.edgexpu_gguf_tensor_elements(None) == 0
    k.edgexpu_gguf_dequantize_row.restype = C.c_int
    k.edgexpu_gguf_dequantize_row.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_int, C.c_void_p, C.c_char_p,
                                               C.c_size_t]
    src = (C.c_uint8 * 64)()
    dst = (C.c_float * 256)()
    err = C.create_string_buffer(256)
    t = _tensor(12, (256, 4))
    assert k.edgexpu_gguf_dequantize_row(src, C.byref(t), 4, 256, dst, err, 256) == 0
    assert err.value.decode() == "tensor 行越界"
    assert k.edgexpu_gguf_dequantize_row(src, C.byref(t), 0, 300, dst, err, 256) == 0
    assert err.value.decode() == "tensor 行宽与 embedding_length 不匹配"
    assert k.edgexpu_gguf_dequantize_row(None, C.byref(t), 0, 256, dst, err, 256) == 0
    assert err.value.decode() == "dequantize_row 参数为空"
    k.edgexpu_gguf_dequantize_q8_0_rows.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_void_p]
    assert k.edgexpu_gguf_dequantize_q8_0_rows(src, 0, 48, dst) == 0      # not whole blocks
    k.edgexpu_gguf_q8_0_dot_row.restype = C.c_float
    k.edgexpu_gguf_q8_0_dot_row.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_void_p]
    assert k.edgexpu_gguf_q8_0_dot_row(src, 0, 33, dst) == 0.0


def test_sampling_argument_checks_without_gpu():
    """edgexpu_cpu_sample_softmax / edgexpu_cpu_softmax refuse bad arguments
    before any device call, as src/cpu_kernel.c:333-335 and 776-778: 0 and
    nothing written."""
    lib = C.CDLL(E.KERNELS_SO)
    f32p = C.POINTER(C.c_float)
    lib.edgexpu_cpu_sample_softmax.restype = C.c_int
    lib.edgexpu_cpu_sample_softmax.argtypes = [f32p, C.c_int, C.c_float, C.POINTER(C.c_uint64),
                                               C.POINTER(C.c_uint32)]
    lib.edgexpu_cpu_softmax.restype = None
    lib.edgexpu_cpu_softmax.argtypes = [f32p, C.c_int]
    io = np.ones(4, np.float32)
    st, out = C.c_uint64(5), C.c_uint32(9)
    p = io.ctypes.data_as(f32p)
    assert lib.edgexpu_cpu_sample_softmax(p, 0, 1.0, C.byref(st), C.byref(out)) == 0
    assert lib.edgexpu_cpu_sample_softmax(p, -3, 0.5, C.byref(st), C.byref(out)) == 0
    assert lib.edgexpu_cpu_sample_softmax(None, 4, 1.0, C.byref(st), C.byref(out)) == 0
    assert lib.edgexpu_cpu_sample_softmax(p, 4, 1.0, None, C.byref(out)) == 0
    assert lib.edgexpu_cpu_sample_softmax(p, 4, 1.0, C.byref(st), None) == 0
    lib.edgexpu_cpu_softmax(None, 4)
    lib.edgexpu_cpu_softmax(p, 0)
    assert st.value == 5 and out.value == 9 and np.array_equal(io, np.ones(4, np.float32))


def test_registry_refusals_without_gpu():
    """edgexpu_kernels_register_weight refuses a NULL weight before any device
    work; lookup and unregister of a pointer never registered find nothing."""
    k = C.CDLL(E.KERNELS_SO)
    k.edgexpu_kernels_register_weight.restype = C.c_int
    k.edgexpu_kernels_register_weight.argtypes = [C.c_void_p, C.c_uint32, C.c_int, C.c_int, C.c_void_p]
    k.edgexpu_kernels_unregister_weight.restype = C.c_int
    k.edgexpu_kernels_unregister_weight.argtypes = [C.c_void_p]
    k.edgexpu_kernels_lookup_weight.restype = C.c_void_p
    k.edgexpu_kernels_lookup_weight.argtypes = [C.c_void_p]
    assert k.edgexpu_kernels_register_weight(None, 12, 4, 256, None) == 0
    buf = C.create_string_buffer(16)
    assert k.edgexpu_kernels_lookup_weight(C.addressof(buf)) is None
    assert k.edgexpu_kernels_unregister_weight(C.addressof(buf)) == 0
    assert k.edgexpu_kernels_unregister_weight(None) == 0


REF_INCLUDE = "/root/reference/include"


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="the reference's headers are absent")
def test_drop_in_header_compiles_with_reference_headers(tmp_path):
    """A C translation unit that includes the reference's own gguf_quant.h and
    cpu_kernel.h together with include/edgexpu_kernels.h compiles under
    -Wall -Wextra -Werror (every function both declare has the same
    signature), and links against libedgexpu_kernels.so with every
    reference-named entry point resolved there."""
    import subprocess

    names = ["edgexpu_cpu_linear_quant", "edgexpu_cpu_linear_quant_batch", "edgexpu_cpu_softmax",
             "edgexpu_cpu_sample_softmax"] + [n for n in declared("edgexpu_kernels.h") if n.startswith("edgexpu_gguf_")]
    src = tmp_path / "dropin.c"
    src.write_text(
        "#include \"edgexpu/gguf_quant.h\"\n#include \"edgexpu/cpu_kernel.h\"\n#include \"edgexpu_kernels.h\"\n"
        "#include <stdio.h>\n"
        "int main(void) {\n    void (*volatile fns[])(void) = {\n"
        + "".join(f"        (void (*)(void)){n},\n" for n in names)
        + "    };\n    printf(\"%p\\n\", (void *)fns[0]);\n    return 0;\n}\n")
    obj, exe = tmp_path / "dropin.o", tmp_path / "dropin"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-Wno-cast-function-type", "-I", REF_INCLUDE,
                    "-I", os.path.join(ROOT, "include"), "-c", str(src), "-o", str(obj)], check=True)
    libdir = os.path.dirname(E.KERNELS_SO)
    subprocess.run(["gcc", str(obj), "-o", str(exe), "-L", libdir, "-ledgexpu_kernels",
                    "-Wl,--allow-shlib-undefined", "-Wl,--no-undefined"], check=True)
