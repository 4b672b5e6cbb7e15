"""The Rust binding a maintainer drops into Atlas (crates/atlas-hip-ops):
no Rust toolchain is present here, so these CPU checks parse the crate's
source.  Its `extern "C"` block declares every C entry point of
include/atlas_hip_ops.h and include/atlas_gguf.h with the same arity and the
same pointer constness (and gen_ffi.py reproduces the committed file); the
safe layer calls only declared functions and keeps atlas_ops::NeuralOps's
method names (crates/atlas-ops/src/lib.rs:20-147)."""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "crates", "atlas-hip-ops")
HEADERS = [os.path.join(ROOT, "include", h) for h in ("atlas_hip_ops.h", "atlas_gguf.h")]


def header_prototypes():
    """{name: [param C type text]} from the headers (comments stripped)."""
    out = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"\b(atlas_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            params = " ".join(m.group(2).split())
            out[m.group(1)] = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
    return out


def rust_externs():
    """{name: [param Rust type text]} from the extern block of src/ffi.rs."""
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (atlas_\w+)\(([^)]*)\)", block):
        params = m.group(2).strip()
        out[m.group(1)] = [] if not params else [p.split(":", 1)[1].strip() for p in params.split(",")]
    return out


def test_ffi_declares_every_entry_point_with_its_arity():
    c, rs = header_prototypes(), rust_externs()
    assert len(c) >= 80
    assert set(c) == set(rs), set(c) ^ set(rs)
    for name, params in c.items():
        assert len(params) == len(rs[name]), name


def test_ffi_pointer_constness_and_widths_match():
    widths = {"float": "f32", "double": "f64", "size_t": "usize", "uint8_t": "u8", "uint16_t": "u16",
              "uint32_t": "u32", "uint64_t": "u64", "int64_t": "i64", "int": "c_int"}
    c, rs = header_prototypes(), rust_externs()
    for name, params in c.items():
        for cp, rp in zip(params, rs[name]):
            stars = cp.count("*")
            assert rp.count("*") == stars, (name, cp, rp)
            if stars:
                # `const T **` is a mutable pointer to a pointer to const T:
                # the outer levels are *mut, the innermost carries the const
                ptrs = rp.split()[:stars]
                assert ptrs[:-1] == ["*mut"] * (stars - 1), (name, cp, rp)
                assert ptrs[-1] == ("*const" if cp.startswith("const") else "*mut"), (name, cp, rp)
            else:
                base = cp.split()[-2] if len(cp.split()) > 1 else cp
                assert widths.get(base) == rp, (name, cp, rp)


def test_generated_file_is_current():
    rc = subprocess.run([sys.executable, os.path.join(CRATE, "gen_ffi.py"), "--check"]).returncode
    assert rc == 0, "src/ffi.rs differs from the headers: run crates/atlas-hip-ops/gen_ffi.py"


def test_safe_layer_calls_declared_functions_and_mirrors_neural_ops():
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    declared = set(rust_externs())
    called = set(re.findall(r"ffi::(atlas_\w+)", lib))
    assert called and called <= declared, called - declared
    # atlas_ops::NeuralOps's methods (crates/atlas-ops/src/lib.rs:34-83) that this path covers
    impl = lib[lib.index("impl NeuralOps {"):]
    for method in ("new", "runtime", "embedding", "add", "multiply", "silu", "rms_norm", "rope"):
        assert re.search(rf"pub fn {method}\(", impl), method
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=atlas_hip_ops" in build
    assert 'links = "atlas_hip_ops"' in open(os.path.join(CRATE, "Cargo.toml")).read()


def test_safe_resident_ops_check_buffer_lengths():
    """Every safe method of HipRuntime that enqueues a kernel checks each
    buffer it passes against the elements the op touches (`holds`) before
    the FFI call, and device buffers hold only the sealed plain-data types
    (no `T: Copy` bound that would admit bool, enums or padded structs)."""
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    impl = lib[lib.index("impl HipRuntime {"):lib.index("impl Drop for HipRuntime")]
    ops = re.split(r"\n    pub fn ", impl)[1:]
    enqueuing = [m for m in ops if re.search(r"ffi::atlas_hip_(rms|add_rms|qk|swiglu|geglu|embed|ple)", m)
                 or "atlas_hip_embed_q" in m or "atlas_hip_ple_q" in m]
    assert len(enqueuing) >= 9, len(enqueuing)
    for body in enqueuing:
        name = body.split("(", 1)[0]
        call = body.index("self.check(")
        assert "holds(" in body[:call], f"{name} calls the library before checking its buffers"
        params = re.findall(r"(\w+): (?:Option<)?&DeviceBuffer", body.split(") ->", 1)[0])
        for p in params:
            assert re.search(rf"holds\({p}\b|Some\(b\) = {p}", body[:call]), (name, p)
    assert "T: Copy" not in lib
    assert re.search(r"pub trait DevicePod: Copy \+ sealed::Sealed \{\}", lib)
