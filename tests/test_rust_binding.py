"""The Rust drop-in (integration/ppk_ffi.rs and the ROCm ops files
integration/int8_kv_ops_rocm.rs, hip_attention_rocm.rs, hip_sampling_rocm.rs)
against the C header, without a Rust toolchain (there is none in this image).

* every argument struct of include/ppk_int8_kv.h has a #[repr(C)] twin with
  the same fields in the same order, each of the Rust type the C type maps to;
* the offsets and sizes those Rust types give under C layout rules equal the
  C compiler's offsetof / sizeof;
* every PPK_API function has an extern "C" declaration with the same
  parameters (pointer constness included) and return type;
* the constants carry the header's values;
* the ROCm ops files use only names ppk_ffi.rs defines and only fields of the
  argument block each variable holds.
"""
from __future__ import annotations

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ppk_int8_kv.h")
FFI = os.path.join(ROOT, "integration", "ppk_ffi.rs")
OPS = os.path.join(ROOT, "integration", "int8_kv_ops_rocm.rs")
FLOAT_OPS = os.path.join(ROOT, "integration", "hip_attention_rocm.rs")
SAMPLER_OPS = os.path.join(ROOT, "integration", "hip_sampling_rocm.rs")
ALL_OPS = (OPS, FLOAT_OPS, SAMPLER_OPS)

C_SCALARS = {"uint32_t": "u32", "int32_t": "i32", "uint64_t": "u64", "float": "f32", "double": "f64",
             "uint8_t": "u8", "char": "c_char", "void": "c_void"}
RUST_SIZES = {"u32": 4, "i32": 4, "u64": 8, "f32": 4, "f64": 8, "u8": 1, "c_char": 1}


def _strip_c_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _c_type_to_rust(tokens: list[str]) -> str:
    """['const', 'ppk_kv_cache', '*', 'const', '*'] -> '*const *const ppk_kv_cache' (C reads right to left)."""
    i, base_const = 0, False
    if tokens[i] == "const":
        base_const, i = True, i + 1
    base = tokens[i]
    i += 1
    if i < len(tokens) and tokens[i] == "const":
        base_const, i = True, i + 1
    rust, pointee_const = C_SCALARS.get(base, base), base_const
    while i < len(tokens):
        assert tokens[i] == "*", tokens
        rust = ("*const " if pointee_const else "*mut ") + rust
        i += 1
        pointee_const = False
        if i < len(tokens) and tokens[i] == "const":
            pointee_const, i = True, i + 1
    return rust


def _c_decl(decl: str) -> tuple[str, str]:
    """'const uint32_t* past' -> ('past', '*const u32'); 'char format[64]' -> ('format', '[c_char; 64]')."""
    decl = decl.strip()
    arr = re.match(r"(.*?)\[(\d+)\]$", decl)
    n = None
    if arr:
        decl, n = arr.group(1).strip(), int(arr.group(2))
    tokens = re.findall(r"\*|\w+", decl)
    name, ty = tokens[-1], _c_type_to_rust(tokens[:-1])
    return name, (f"[{ty}; {n}]" if n is not None else ty)


def header_structs() -> dict[str, list[tuple[str, str]]]:
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for name, body in re.findall(r"typedef struct (\w+) \{(.*?)\} \1;", text, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            first, *more = [d.strip() for d in decl.split(",")]
            fields.append(_c_decl(first))
            base = re.match(r"((?:const\s+)?\w+)", first).group(1)
            fields += [_c_decl(f"{base} {d}") for d in more]
        out[name] = fields
    return out


def header_functions() -> dict[str, tuple[str, list[str]]]:
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"PPK_API\s+([\w\s\*]+?)\s*\b(ppk_\w+)\s*\(([^)]*)\)\s*;", text):
        ret_rust = _c_type_to_rust(re.findall(r"\*|\w+", ret))
        plist = [] if params.strip() == "void" else [_c_decl(" ".join(p.split()))[1] for p in params.split(",")]
        out[name] = (ret_rust, plist)
    return out


def header_constants() -> dict[str, int]:
    text = _strip_c_comments(open(HEADER).read())
    consts = {k: int(v) for k, v in re.findall(r"\b(PPK_\w+)\s*=\s*(\d+)u?\b", text)}
    for k, v in re.findall(r"#define (PPK_\w+) (\(?[\d u<>]+\)?)\s*$", text, flags=re.M):
        consts[k] = eval(re.sub(r"(\d+)u", r"\1", v))  # integer literals and shifts only
    return consts


def _rust_text(path: str) -> str:
    return re.sub(r"//[^\n]*", "", open(path).read())


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    text = _rust_text(FFI)
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*(?:#\[derive\([^\]]*\)\]\s*)?pub struct (\w+)\s*\{(.*?)\}",
                                 text, flags=re.S):
        fields = re.findall(r"(?:pub\s+)?(\w+)\s*:\s*([^,]+?)\s*,", body + ",")
        out[name] = [(f, " ".join(t.split())) for f, t in fields]
    return out


def rust_functions() -> dict[str, tuple[str, list[str]]]:
    text = _rust_text(FFI)
    block = re.search(r'extern "C" \{(.*?)\n\}', text, flags=re.S).group(1)
    out = {}
    for name, params, ret in re.findall(r"pub fn (\w+)\s*\(([^)]*)\)\s*->\s*([^;]+);", block, flags=re.S):
        plist = [" ".join(p.split(":", 1)[1].split()) for p in params.split(",") if p.strip()]
        out[name] = (" ".join(ret.split()), plist)
    return out


def rust_constants() -> dict[str, int]:
    text = _rust_text(FFI)
    return {k: eval(v) for k, v in re.findall(r"pub const (PPK_\w+): \w+ = ([\d <>]+);", text)}


def _layout(ty: str, structs: dict) -> tuple[int, int]:
    """(size, align) of a Rust FFI type under C rules (x86-64 / amdgcn LP64)."""
    if ty.startswith("*"):
        return 8, 8
    arr = re.match(r"\[(.+); (\d+)\]$", ty)
    if arr:
        size, align = _layout(arr.group(1), structs)
        return size * int(arr.group(2)), align
    if ty in RUST_SIZES:
        return RUST_SIZES[ty], RUST_SIZES[ty]
    offsets, size, align = _offsets(structs[ty], structs)
    return size, align


def _offsets(fields, structs) -> tuple[dict[str, int], int, int]:
    off, align, out = 0, 1, {}
    for name, ty in fields:
        size, a = _layout(ty, structs)
        off = -(-off // a) * a
        out[name] = off
        off += size
        align = max(align, a)
    return out, -(-off // align) * align, align


@pytest.fixture(scope="module")
def c_offsets(tmp_path_factory):
    structs = header_structs()
    src = tmp_path_factory.mktemp("rust_abi") / "layout.c"
    exe = src.with_suffix("")
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    for name, fields in structs.items():
        lines.append(f'printf("{name} __sizeof__ %zu\\n", sizeof({name}));')
        for field, _ in fields:
            lines.append(f'printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return {tuple(line.split()[:2]): int(line.split()[2]) for line in out.splitlines()}


def test_header_parser_sees_every_struct():
    names = set(header_structs())
    assert names == {"PpkQuantizeArgs", "PpkAppendArgs", "PpkDequantizeArgs", "PpkAttentionArgs",
                     "PpkDecodeStepArgs", "PpkFloatAttentionArgs", "PpkFloatDecodeStepArgs", "PpkRenyiSampleArgs",
                     "PpkKvConfig", "PpkKvView", "PpkKvInfo", "PpkKvWrite", "PpkInt8KvStatus", "PpkAttentionPlanInfo"}
    # The multi-declarator line of PpkAppendArgs and the trailing optional field of PpkAttentionArgs.
    append = dict(header_structs()["PpkAppendArgs"])
    assert [append[k] for k in ("batch", "heads", "tokens", "head_dim", "capacity")] == ["u32"] * 5
    assert header_structs()["PpkAttentionArgs"][-1] == ("past_host", "*const u32")


@pytest.mark.parametrize("name", sorted(header_structs()))
def test_rust_struct_fields_match_the_header(name):
    rust = rust_structs()
    assert name in rust, f"ppk_ffi.rs lacks #[repr(C)] {name}"
    assert rust[name] == header_structs()[name]


@pytest.mark.parametrize("name", sorted(header_structs()))
def test_rust_struct_layout_matches_c(c_offsets, name):
    rust = rust_structs()
    offsets, size, _ = _offsets(rust[name], rust)
    assert size == c_offsets[(name, "__sizeof__")], f"sizeof {name}"
    for field, off in offsets.items():
        assert off == c_offsets[(name, field)], f"{name}.{field}"


def test_opaque_handles_are_declared():
    rust = rust_structs()
    for handle in ("ppk_context", "ppk_kv_cache", "ppk_write_plan"):
        assert rust[handle] == [("_opaque", "[u8; 0]")]


def test_every_function_is_declared_with_the_same_signature():
    c, rust = header_functions(), rust_functions()
    assert len(c) >= 30
    assert sorted(c) == sorted(rust), "extern block differs from the header's PPK_API list"
    for name, (ret, params) in c.items():
        assert rust[name] == (ret, params), name


def test_constants_match_the_header():
    c, rust = header_constants(), rust_constants()
    assert c["PPK_FLAG_STALE_LENGTHS"] == 4 and c["PPK_NOALLOC_SCRATCH_BYTES"] == 8 << 20
    assert sorted(c) == sorted(rust)
    for k, v in c.items():
        assert rust[k] == v, k


def _declared() -> set[str]:
    ffi_text = _rust_text(FFI)
    declared = set(rust_functions()) | set(rust_constants()) | set(rust_structs())
    for kind in ("fn", "struct", "const"):
        declared |= set(re.findall(rf"^pub {kind} (\w+)", ffi_text, flags=re.M))
    return declared


@pytest.mark.parametrize("path", ALL_OPS, ids=os.path.basename)
def test_rocm_ops_use_only_declared_names(path):
    ops = _rust_text(path)
    used = set(re.findall(r"(?<!std::)\bffi::(\w+)", ops)) - {"c_void"}  # std::ffi's, imported by name
    for names in re.findall(r"use crate::model::ppk_ffi::\{([^}]*)\};", ops):
        used |= {n.strip() for n in names.split(",") if n.strip()}
    assert used and used <= _declared(), sorted(used - _declared())
    # Helpers imported by name are used (and so checked for their declaration above).
    for names in re.findall(r"use crate::model::ppk_ffi::\{([^}]*)\};", ops):
        for name in (n.strip() for n in names.split(",") if n.strip()):
            assert len(re.findall(rf"\b{name}\b", ops)) > 1, f"{name} imported but unused"


def test_rocm_ops_set_only_fields_of_their_argument_blocks():
    # Each argument block is built by ffi::args() and only its own fields are set (checked per function body,
    # where the variable names are bound).
    structs = rust_structs()
    seen = set()
    for path in ALL_OPS:
        for body in re.split(r"\n\s*(?:pub(?:\((?:super|crate)\))? )?fn ", _rust_text(path))[1:]:
            for var, ty in re.findall(r"let mut (\w+): ffi::(\w+) = ffi::args\(\);", body):
                seen.add(ty)
                fields = {f for f, _ in structs[ty]}
                for field in re.findall(rf"\b{var}\.(\w+)\s*=", body):
                    assert field in fields, f"{os.path.basename(path)}: {ty}.{field}"
    assert seen == {"PpkQuantizeArgs", "PpkDequantizeArgs", "PpkAttentionArgs", "PpkDecodeStepArgs",
                    "PpkAppendArgs", "PpkFloatAttentionArgs", "PpkFloatDecodeStepArgs", "PpkRenyiSampleArgs"}


def test_rocm_ops_cover_the_reference_functions():
    ops = _rust_text(OPS)
    # Every ROCm branch the header's int8 entry points replace is present.
    for fn in ("quantize", "dequantize", "attention", "decode_step", "commit_append", "prepare"):
        assert re.search(rf"pub\(super\) fn {fn}\(", ops), fn
    for call in ("ppk_quantize", "ppk_dequantize", "ppk_decode_attention", "ppk_decode_step",
                 "ppk_quantize_append", "ppk_prepare", "ppk_attention_workspace_bytes"):
        assert f"ffi::{call}(" in ops, call
    # hip_attention.rs's three functions (hip_attention.rs:7,18,47) with the reference's visibility.
    fl = _rust_text(FLOAT_OPS)
    for vis, fn in (("crate", "prepare"), ("crate", "validate_split_k"), ("super", "decode_attention"),
                    ("super", "decode_attention_with_host_lengths"), ("super", "decode_step")):
        assert re.search(rf"pub\({vis}\) fn {fn}\(", fl), fn
    for call in ("ppk_float_decode_attention", "ppk_float_attention_plan", "ppk_float_attention_prepare",
                 "ppk_float_decode_step"):
        assert f"ffi::{call}(" in fl, call
    # HipSampler::rocm_fwd's body (hip_sampling.rs:120-214).
    sm = _rust_text(SAMPLER_OPS)
    assert re.search(r"pub\(super\) fn rocm_fwd\(\s*op: &super::HipSampler,", sm)
    assert "ffi::ppk_renyi_sample(" in sm
