"""INTEGRATION.md's Rust binding, held to the C header on the CPU (the image has no rustc).

The `-sys` block must restate `include/staleynet_gemm.h` exactly:
- every `#define SN_*` as a `pub const` of the same value and width;
- every struct with the same field names, order and C widths, with a `#[repr(C)]` layout whose size is
  the ctypes mirror's;
- every function with the same name, argument types and result.

The shim must use only `sys::` names that block defines. It must keep the reference's interface:
- `GpuResult<T> = Result<T, DriverError>` (crates/staleynet-cuda/src/device.rs:12);
- the public `matmul_kernel` field (device.rs:144), which `Gpu::matmul` reads on every call, as
  ops/matmul.rs:151 does and as kernels_match_reference.rs:77, staleynet-cli train.rs:111 and
  bench.rs:289 rely on when they assign it;
- the reference's three matmul panics (ops/matmul.rs:147-149).
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "staleynet_gemm.h")
INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")

C_SCALARS = {"size_t": "usize", "uint32_t": "u32", "uint64_t": "u64", "float": "f32", "int": "c_int",
             "void": "c_void", "char": "c_char"}
RUST_SIZES = {"usize": 8, "u64": 8, "u32": 4, "f32": 4, "c_int": 4}


def strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", " ", text, flags=re.S)


def strip_rust_comments(text):
    return re.sub(r"//[^\n]*", "", text)


@pytest.fixture(scope="module")
def header():
    return strip_c_comments(open(HEADER).read())


@pytest.fixture(scope="module")
def rust_blocks():
    return re.findall(r"```rust\n(.*?)```", open(INTEGRATION).read(), flags=re.S)


@pytest.fixture(scope="module")
def sys_block(rust_blocks):
    blocks = [b for b in rust_blocks if "crates/staleynet-gemm-sys/src/lib.rs" in b]
    assert len(blocks) == 1
    return strip_rust_comments(blocks[0])


def c_value(text):
    text = text.replace("(size_t)", "").replace("u", "").strip()
    assert re.fullmatch(r"[0-9A-Fa-fx()<\- ]+", text), text
    return eval(text)  # digits, hex, parentheses, shifts and minus only (checked above)


def rust_value(text):
    text = text.replace("_", "").strip()
    assert re.fullmatch(r"[0-9A-Fa-fx()<\- ]+", text), text
    return eval(text)


def header_constants(header):
    out = {}
    for name, value in re.findall(r"#define (SN_\w+) ([^\n]+)", header):
        v = value.strip()
        width = "usize" if "size_t" in v else "u32" if v.endswith("u") else "c_int"
        out[name] = (c_value(v), width)
    return out


def rust_constants(block):
    return {name: (rust_value(value), kind) for name, kind, value in
            re.findall(r"pub const (\w+): (\w+) = ([^;]+);", block)}


def c_type_to_rust(c_type):
    """`const float *` -> `*const f32`, `float **` -> `*mut *mut f32`, `size_t` -> `usize`."""
    t = c_type.strip()
    stars = t.count("*")
    base_const = t.startswith("const ")
    base = t.replace("const ", "").replace("*", "").strip()
    rust = C_SCALARS.get(base, base)
    if stars == 0:
        return rust
    out = ("*const " if base_const else "*mut ") + rust
    for _ in range(stars - 1):
        out = "*mut " + out
    return out


def split_params(params):
    params = params.strip()
    if not params or params == "void":
        return []
    return [p.strip() for p in params.split(",")]


def header_functions(header):
    out = {}
    for ret, name, params in re.findall(r"^((?:const )?\w+ \*?)(sn_\w+)\(([^;]*?)\);", header, flags=re.M | re.S):
        types = []
        for p in split_params(" ".join(params.split())):
            m = re.fullmatch(r"(.*?)(\w+)", p)
            types.append(c_type_to_rust(m.group(1)))
        out[name] = (c_type_to_rust(ret), types)
    return out


def rust_functions(block):
    out = {}
    for name, params, ret in re.findall(r"pub fn (sn_\w+)\((.*?)\)\s*->\s*([^;]+);", block, flags=re.S):
        types = [" ".join(p.split(":", 1)[1].split()) for p in split_params(" ".join(params.split()))]
        out[name] = (" ".join(ret.split()), types)
    return out


def header_structs(header):
    out = {}
    for name, body in re.findall(r"typedef struct (sn_\w+) \{(.*?)\} \1;", header, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            c_type, names = decl.split(" ", 1)
            fields += [(n.strip(), C_SCALARS[c_type]) for n in names.split(",")]
        out[name] = fields
    return out


def rust_structs(block):
    out = {}
    for attrs, name, body in re.findall(r"((?:#\[[^\]]*\]\s*)*)pub struct (sn_\w+) \{(.*?)\}", block, flags=re.S):
        assert "#[repr(C)]" in attrs, f"{name} lacks #[repr(C)]"
        if name != "sn_context":  # the opaque handle, checked on its own
            out[name] = re.findall(r"pub (\w+): (\w+)", body)
    return out


def repr_c_size(fields):
    offset, align = 0, 1
    for _, t in fields:
        size = RUST_SIZES[t]
        offset = (offset + size - 1) // size * size + size
        align = max(align, size)
    return (offset + align - 1) // align * align


def test_every_header_constant_is_defined_with_its_value_and_width(header, sys_block):
    want, got = header_constants(header), rust_constants(sys_block)
    assert set(got) == set(want), (sorted(set(want) - set(got)), sorted(set(got) - set(want)))
    for name, (value, width) in want.items():
        assert got[name] == (value, width), (name, got[name], (value, width))


def test_every_struct_matches_the_header_field_for_field(header, sys_block):
    from staleynet_amd import gemm

    want, got = header_structs(header), rust_structs(sys_block)
    assert set(want) == {"sn_matmul_spec", "sn_head_layout", "sn_attention_shape", "sn_cross_entropy_head",
                         "sn_launch_plan"}
    assert set(got) == set(want)
    for name in want:
        assert got[name] == want[name], name
    mirrors = {"sn_matmul_spec": gemm.CMatmulSpec, "sn_head_layout": gemm.CHeadLayout,
               "sn_attention_shape": gemm.CAttentionShape, "sn_cross_entropy_head": gemm.CCrossEntropyHead,
               "sn_launch_plan": gemm.CLaunchPlan}
    for name, mirror in mirrors.items():
        assert repr_c_size(got[name]) == ctypes.sizeof(mirror), name
    assert re.search(r"#\[repr\(C\)\]\s*pub struct sn_context \{\s*_private: \[u8; 0\],\s*\}", sys_block)


def test_every_function_matches_the_header_signature(header, sys_block):
    want, got = header_functions(header), rust_functions(sys_block)
    assert len(want) >= 39
    assert set(got) == set(want), (sorted(set(want) - set(got)), sorted(set(got) - set(want)))
    for name, (ret, params) in want.items():
        assert got[name] == (ret, params), (name, got[name], (ret, params))


def test_the_shim_uses_only_names_the_sys_block_defines(rust_blocks, sys_block):
    defined = set(rust_constants(sys_block)) | set(rust_functions(sys_block)) | set(rust_structs(sys_block)) | \
        {"sn_context"}
    used = set()
    for block in rust_blocks:
        used |= set(re.findall(r"sys::(\w+)", strip_rust_comments(block)))
    assert used, "the shim calls nothing"
    assert used <= defined, sorted(used - defined)


def test_the_shim_keeps_the_reference_result_type_and_kernel_field(rust_blocks):
    text = "\n".join(strip_rust_comments(b) for b in rust_blocks)
    doc = open(INTEGRATION).read()
    # No error type the reference does not have (its GpuResult is Result<T, DriverError>).
    assert "GpuError" not in doc
    assert "pub type GpuResult<T = ()> = Result<T, DriverError>;" in text
    assert re.search(r"pub struct DriverError\(pub c_int\);", text)
    assert "impl std::error::Error for DriverError {}" in text
    # The public field, and Gpu::matmul pushing it before every product.
    assert re.search(r"pub struct Gpu \{[^}]*pub matmul_kernel: MatmulKernel,", text, flags=re.S)
    body = re.search(r"pub fn matmul\(&self, spec: &MatmulSpec, left: &Tensor, right: &Tensor, "
                     r"output: &mut Tensor\) -> GpuResult \{(.*?)\n    \}\n", text, flags=re.S)
    assert body, "Gpu::matmul with the reference's signature (ops/matmul.rs:146)"
    body = body.group(1)
    set_kernel = body.find("sys::sn_context_set_kernel(self.raw(), self.matmul_kernel.ffi())")
    assert 0 <= set_kernel < body.find("sys::sn_matmul("), "the kernel is pushed before the product"
    for message in ("matmul: left operand too small", "matmul: right operand too small", "matmul: output too small"):
        assert f'panic!("{message}")' in body
    # MatmulKernel's four variants map onto the library's three kernels.
    for variant, kernel in (("MatmulKernel::Naive | MatmulKernel::Tiled", "SN_KERNEL_SIMPLE"),
                            ("MatmulKernel::Blocked", "SN_KERNEL_MFMA_F32"),
                            ("MatmulKernel::TensorCore", "SN_KERNEL_MFMA_BF16")):
        assert f"{variant} => sys::{kernel}," in text
    assert "unsafe { sys::sn_kernel_tolerance(self.ffi()) }" in text


def test_the_parser_catches_a_planted_mismatch(header, sys_block):
    # A wrong value, a dropped field and a wrong argument type must each fail the comparisons above.
    constants = rust_constants(sys_block.replace("pub const SN_ERR_SHAPE: c_int = -12;",
                                                 "pub const SN_ERR_SHAPE: c_int = -13;"))
    assert constants["SN_ERR_SHAPE"] != header_constants(header)["SN_ERR_SHAPE"]
    structs = rust_structs(re.sub(r"pub query_offset: usize,", "", sys_block, count=1))
    assert structs["sn_matmul_spec"] != header_structs(header)["sn_matmul_spec"]
    functions = rust_functions(sys_block.replace("pub fn sn_free(context: *mut sn_context, buffer: *mut f32)",
                                                 "pub fn sn_free(context: *mut sn_context, buffer: *const f32)"))
    assert functions["sn_free"] != header_functions(header)["sn_free"]
