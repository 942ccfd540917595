"""The Rust crate integration/ffai-hip against the C headers, on the CPU (no Rust toolchain is
needed): every function include/*.h declares is declared in src/ffi.rs with the same number of
arguments, every struct has the same fields in the same order, and build.rs compiles the same
sources with the same device flags as ffai_amd/build.py."""

from __future__ import annotations

import os
import re

from ffai_amd import build as native_build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "integration", "ffai-hip")


def _strip_c(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _c_functions() -> dict:
    out = {}
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not fn.endswith(".h"):
            continue
        text = _strip_c(open(os.path.join(ROOT, "include", fn)).read())
        for m in re.finditer(r"\b(ffai_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            args = m.group(2).strip()
            out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _rust_functions() -> dict:
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    text = re.sub(r"//[^\n]*", "", text)
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (ffai_[a-z0-9_]+)\s*\(([^)]*)\)", block, flags=re.S):
        args = m.group(2).strip().rstrip(",")
        out[m.group(1)] = 0 if not args else args.count(",") + 1
    return out


def _c_structs() -> dict:
    out = {}
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not fn.endswith(".h"):
            continue
        text = _strip_c(open(os.path.join(ROOT, "include", fn)).read())
        for m in re.finditer(r"typedef struct (ffai_[a-z0-9_]+) \{(.*?)\} \1;", text, flags=re.S):
            fields = []
            for decl in m.group(2).split(";"):
                decl = decl.strip()
                if not decl:
                    continue
                head, *names = [x.strip() for x in decl.split(",")]
                first = head.split()[-1].lstrip("*")
                for name in [first] + [n.lstrip("*") for n in names]:
                    fields.append(re.sub(r"\[.*\]", "", name))
            out[m.group(1)] = fields
    return out


def _rust_structs() -> dict:
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"pub struct (ffai_[a-z0-9_]+) \{(.*?)\}", text, flags=re.S):
        out[m.group(1)] = re.findall(r"pub (\w+):", m.group(2))
    return out


def test_every_header_function_is_declared_with_its_arity():
    c, r = _c_functions(), _rust_functions()
    assert len(c) >= 30
    assert sorted(c) == sorted(r), (set(c) ^ set(r))
    for name, n in c.items():
        assert r[name] == n, (name, n, r[name])


def test_structs_have_the_same_fields_in_order():
    c, r = _c_structs(), _rust_structs()
    assert set(c) == {"ffai_attn_desc", "ffai_tensor", "ffai_kv_cache", "ffai_encoder_attn_desc",
                      "ffai_encoder_attn_weights"}
    for name, fields in c.items():
        assert r[name] == fields, (name, fields, r[name])


def test_build_script_matches_the_native_build():
    text = open(os.path.join(CRATE, "build.rs")).read()
    listed = re.search(r"const SOURCES: \[&str; (\d+)\] = \[(.*?)\];", text, flags=re.S)
    names = re.findall(r'"([^"]+)"', listed.group(2))
    assert int(listed.group(1)) == len(names)
    assert names == [os.path.basename(s) for s in native_build.SOURCES]
    # the device-only NaN assumptions and the packed-FP32 switch, as ffai_amd/build.py passes them
    flags = native_build.flags()
    for pair in (("-Xarch_device", "-fno-honor-nans"), ("-Xarch_device", "-mno-amdgpu-ieee")):
        assert any(flags[i:i + 2] == list(pair) for i in range(len(flags) - 1))
        assert '"{}", "{}"'.format(*pair) in text
    assert '"-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"' in text
    assert "--offload-arch=gfx950" in text
