"""The Rust crate's FFI (marian-edge_amd/rust/marian-hip/src/ffi.rs) against
the C ABI it binds.  No Rust toolchain is available here, so the crate is
checked by reading it: every struct it mirrors has the header's fields in the
header's order, every function it declares exists in include/*.h with the
same number of parameters and is exported by libmarian_hip.so, the engine-level
entry points are all declared, and the status codes, flags and ABI version
agree with the header's."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CRATE = ROOT / "marian-edge_amd" / "rust" / "marian-hip"
HEADERS = [ROOT / "include" / "marian_hip.h", ROOT / "include" / "marian_hip_util.h"]
ENGINE_LEVEL = {
    "marian_hip_engine_create", "marian_hip_engine_create_ssru", "marian_hip_engine_destroy",
    "marian_hip_translate_token_ids", "marian_hip_translate_shortlisted", "marian_hip_is_ready",
    "marian_hip_last_error", "marian_hip_info", "marian_hip_last_stats", "marian_hip_warmup",
    "marian_hip_reserve",
}


def strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", " ", text, flags=re.S)


def header_structs():
    out = {}
    for h in HEADERS:
        text = strip_c_comments(h.read_text())
        for body, name in re.findall(r"typedef struct \{(.*?)\}\s*(\w+);", text, flags=re.S):
            fields = []
            for decl in body.split(";"):
                decl = decl.strip()
                if not decl:
                    continue
                # "type a, b, c" or "const float* a" -> the declarator names
                m = re.match(r"^(?:const\s+)?[\w]+\s*\**\s*(.*)$", decl, flags=re.S)
                for part in m.group(1).split(","):
                    fields.append(part.strip().lstrip("*").strip())
            out[name] = fields
    return out


def header_functions():
    out = {}
    for h in HEADERS:
        text = strip_c_comments(h.read_text())
        for name, params in re.findall(r"\b(marian_hip_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            p = params.strip()
            out[name] = 0 if p in ("", "void") else p.count(",") + 1
    return out


def rust_structs(src):
    out = {}
    for name, body in re.findall(r"pub struct (\w+)\s*\{(.*?)\n\}", src, flags=re.S):
        out[name] = re.findall(r"pub (\w+):", body)
    return out


def rust_functions(src):
    block = src[src.index('extern "C" {'):]
    out = {}
    for name, params in re.findall(r"pub fn (\w+)\s*\((.*?)\)\s*(?:->[^;]*)?;", block, flags=re.S):
        p = params.strip().rstrip(",")
        out[name] = 0 if not p else p.count(",") + 1
    return out


@pytest.fixture(scope="module")
def ffi_src():
    return (CRATE / "src" / "ffi.rs").read_text()


def test_crate_layout():
    for f in ("Cargo.toml", "build.rs", "src/lib.rs", "src/ffi.rs", "src/engine.rs", "src/model.rs",
              "src/backend.rs"):
        assert (CRATE / f).is_file(), f
    for mod in ("backend", "engine", "ffi", "model"):
        assert f"pub mod {mod};" in (CRATE / "src" / "lib.rs").read_text()


def test_structs_mirror_the_header(ffi_src):
    hs, rs = header_structs(), rust_structs(ffi_src)
    mirrored = [n for n in rs if n in hs]
    assert {"marian_hip_linear", "marian_hip_model", "marian_hip_static_linear",
            "marian_hip_ssru_model", "marian_hip_ssru_encoder_layer", "marian_hip_ssru_decoder_layer",
            "marian_hip_limits", "marian_hip_stats", "marian_hip_encoder_layer",
            "marian_hip_decoder_layer"} <= set(mirrored)
    for n in mirrored:
        assert rs[n] == hs[n], f"{n}: {rs[n]} != {hs[n]}"


def test_functions_exist_with_the_same_arity(ffi_src, pkg):
    hf, rf = header_functions(), rust_functions(ffi_src)
    assert ENGINE_LEVEL <= set(rf), ENGINE_LEVEL - set(rf)
    lib = pkg._lib.load()
    for name, n in rf.items():
        assert name in hf, f"{name} is not declared in include/*.h"
        assert hf[name] == n, f"{name}: {n} parameters in ffi.rs, {hf[name]} in the header"
        assert hasattr(lib, name), f"{name} is not exported by libmarian_hip.so"


def test_constants_agree(ffi_src):
    text = strip_c_comments(HEADERS[0].read_text())
    for c_name, r_name in (("MARIAN_HIP_OK", "OK"), ("MARIAN_HIP_ERR_INVALID_INPUT", "ERR_INVALID_INPUT"),
                           ("MARIAN_HIP_ERR_MODEL", "ERR_MODEL"), ("MARIAN_HIP_ERR_INFERENCE", "ERR_INFERENCE"),
                           ("MARIAN_HIP_ERR_DEVICE", "ERR_DEVICE"), ("MARIAN_HIP_ERR_BUFFER", "ERR_BUFFER"),
                           ("MARIAN_HIP_ERR_NOT_READY", "ERR_NOT_READY")):
        want = int(re.search(rf"{c_name}\s*=\s*(-?\d+)", text).group(1))
        got = int(re.search(rf"pub const {r_name}: c_int = (-?\d+);", ffi_src).group(1))
        assert got == want, c_name
    abi = int(re.search(r"#define MARIAN_HIP_ABI_VERSION (\d+)", text).group(1))
    assert f"pub const MARIAN_HIP_ABI_VERSION: u32 = {abi};" in ffi_src
    assert "pub const FLAG_IGNORE_EOS: u32 = 1 << 0;" in ffi_src
    assert "pub const FLAG_NO_GENERATION_MASK: u32 = 1 << 1;" in ffi_src
