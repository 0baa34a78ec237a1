"""The Rust binding (rust_trainer_amd/rust, a cargo crate: rustc is not in this image, so it is
checked here as text) declares exactly the C ABI of include/rtq.h: every function, with the same
number of parameters, and its FrozenMatmul methods cover the trait (src/frozen.rs:14-25)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "rust_trainer_amd", "rust")


def header_functions():
    text = open(os.path.join(ROOT, "include", "rtq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(rtq_[a-z_0-9]+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def rust_functions():
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (rtq_[a-z_0-9]+)\s*\((.*?)\)\s*(?:->[^;]*)?;", block, flags=re.S):
        args = re.sub(r"\s+", " ", m.group(2)).strip().rstrip(",")
        out[m.group(1)] = 0 if not args else args.count(",") + 1
    return out


def test_rust_ffi_declares_the_whole_header():
    h, r = header_functions(), rust_functions()
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    wrong = {n: (h[n], r[n]) for n in h if h[n] != r[n]}
    assert not wrong, wrong


def test_rust_crate_layout_and_trait_methods():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs"), os.path.join("src", "ffi.rs")):
        assert os.path.exists(os.path.join(CRATE, f)), f
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    macro = lib[lib.index("macro_rules! impl_frozen_matmul"):]
    for method in ("out_dim", "in_dim", "forward", "backward_input", "row", "nbytes"):
        assert f"fn {method}(" in macro
        assert f"pub fn {method}(" in lib
    assert 'links = "rtq"' in open(os.path.join(CRATE, "Cargo.toml")).read()
