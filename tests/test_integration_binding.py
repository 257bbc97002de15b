"""CPU check of the Julia binding written out in INTEGRATION.md against include/reels_hip.h.

Julia is not installed here, so the binding cannot run; this test parses every
``ccall((:symbol, LIB[]), Ret, (types...), args...)`` in the file's Julia code and checks, for
each one, that the symbol is declared in the header, that the return type and every argument
type are the C types the header declares (in order), and that the call passes as many arguments
as it lists types. It also checks that the seams the binding must cover (quantization.jl:54-76,
lora.jl:56-118, ad_rules.jl:55-80) have a method for each activation element type."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")
HEADER = os.path.join(ROOT, "include", "reels_hip.h")

# Julia ccall type -> the C types it may stand for
JULIA_C = {
    "Cint": {"int"},
    "Int64": {"int64_t"},
    "Csize_t": {"size_t"},
    "Cfloat": {"float"},
    "Float32": {"float"},
    "Cstring": {"const char*"},
    "Ptr{Cvoid}": {"void*", "const void*"},
    "Ptr{Int8}": {"int8_t*", "const int8_t*"},
    "Ptr{UInt8}": {"uint8_t*", "const uint8_t*"},
    "Ptr{Int32}": {"int32_t*", "const int32_t*"},
    "Ptr{Float32}": {"float*", "const float*"},
}


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def header_prototypes():
    """{name: (return C type, [param C types])} from the header's declarations."""
    text = _strip_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(reels_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        ret = " ".join(m.group(1).split()).replace(" *", "*")
        params = []
        body = " ".join(m.group(3).split())
        if body and body != "void":
            for p in body.split(","):
                # the type is everything before the parameter name (the last identifier)
                t = re.match(r"^(.*?)[A-Za-z_]\w*\s*$", p.strip()).group(1)
                params.append(re.sub(r"\s*\*\s*", "*", " ".join(t.split())).strip())
        out[m.group(2)] = (ret, params)
    return out


def _split_top(s):
    """Split s on commas outside (), {} and []."""
    parts, depth, cur = [], 0, []
    for ch in s:
        if ch in "({[":
            depth += 1
        elif ch in ")}]":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    tail = "".join(cur).strip()
    if tail:
        parts.append(tail)
    return parts


def _balanced(text, i):
    """Content of the parenthesis opening at text[i]."""
    assert text[i] == "("
    depth = 0
    for j in range(i, len(text)):
        if text[j] == "(":
            depth += 1
        elif text[j] == ")":
            depth -= 1
            if depth == 0:
                return text[i + 1:j]
    raise AssertionError("unbalanced parenthesis in a ccall")


def julia_code():
    doc = open(DOC).read()
    blocks = re.findall(r"```julia\n(.*?)```", doc, flags=re.S)
    assert blocks, "INTEGRATION.md has no Julia code"
    # Julia comments would confuse the splitter (they may hold commas or parentheses)
    return "\n".join(re.sub(r"#[^\n]*", "", b) for b in blocks)


def julia_ccalls():
    code = julia_code()
    calls = []
    for m in re.finditer(r"\bccall\(", code):
        parts = _split_top(_balanced(code, m.end() - 1))
        target, ret, types = parts[0], parts[1], parts[2]
        sym = re.fullmatch(r"\(\s*:(\w+)\s*,\s*LIB\[\]\s*\)", target)
        assert sym, f"ccall target not of the form (:sym, LIB[]): {target}"
        assert types.startswith("(") and types.endswith(")"), types
        tlist = _split_top(types[1:-1])
        calls.append((sym.group(1), ret.strip(), [t.replace(" ", "") for t in tlist], parts[3:]))
    return calls


def test_every_ccall_matches_the_header():
    protos = header_prototypes()
    calls = julia_ccalls()
    assert len(calls) >= 14
    for sym, ret, types, args in calls:
        assert sym in protos, f"{sym} is not declared in reels_hip.h"
        cret, cparams = protos[sym]
        assert cret in JULIA_C[ret], f"{sym}: returns {cret}, ccall says {ret}"
        assert len(types) == len(cparams), \
            f"{sym}: header has {len(cparams)} parameters, ccall lists {len(types)} types"
        for i, (jt, ct) in enumerate(zip(types, cparams)):
            assert jt in JULIA_C, f"{sym}: unknown Julia type {jt}"
            assert ct in JULIA_C[jt], f"{sym} argument {i + 1}: C type {ct}, ccall type {jt}"
        assert len(args) == len(types), \
            f"{sym}: ccall lists {len(types)} types but passes {len(args)} arguments"


def test_binding_covers_the_entry_points_of_every_element_type():
    called = {c[0] for c in julia_ccalls()}
    for sym in ["reels_hip_i8_pack", "reels_hip_i8_dequant", "reels_hip_last_error",
                "reels_hip_i8lora_workspace_bytes", "reels_hip_i8lora_workspace_bytes_f32",
                "reels_hip_i8lora_fwd", "reels_hip_i8lora_fwd_f16", "reels_hip_i8lora_fwd_f32",
                "reels_hip_i8lora_bwd_bias", "reels_hip_i8lora_bwd_bias_f16",
                "reels_hip_i8lora_bwd_bias_f32", "reels_hip_attention_fwd",
                "reels_hip_attention_bwd", "reels_hip_attention_workspace_bytes"]:
        assert sym in called, f"the Julia binding never calls {sym}"


def test_each_element_type_takes_its_own_entry_point():
    """_fwd / _bwd / _ws methods: the element type a method dispatches on names the symbol
    with that type's suffix (none for BFloat16, _f16, _f32)."""
    code = julia_code()
    suffix = {"BFloat16": "", "Float16": "_f16", "Float32": "_f32"}
    base = {"_fwd": "reels_hip_i8lora_fwd", "_bwd": "reels_hip_i8lora_bwd_bias"}
    seen = set()
    for m in re.finditer(r"^(_fwd|_bwd)\(::Type\{(\w+)\}[^=]*=\s*\n?\s*ccall\(\(:(\w+),",
                         code, flags=re.M):
        fn, T, sym = m.groups()
        assert sym == base[fn] + suffix[T], f"{fn}(::Type{{{T}}}) calls {sym}"
        seen.add((fn, T))
    assert seen == {(f, T) for f in base for T in suffix}, seen
    ws = re.findall(r"^_ws\(::Type\{([^}]*)\}\}?[^=]*=\s*\n?\s*ccall\(\(:(\w+),", code, flags=re.M)
    assert ("Float32", "reels_hip_i8lora_workspace_bytes_f32") in ws
    assert any(sym == "reels_hip_i8lora_workspace_bytes" and "Float16" in T for T, sym in ws)


@pytest.mark.parametrize("seam", [
    r"_weight_mul\(W::DevQ, x::ROCMatrix\{T\}\)",
    r"_weight_transpose_mul\(W::DevQ, dy::ROCMatrix\{T\}\)",
    r"_materialize_weight\(W::DevQ, input::ROCArray\{T\}\)",
    r"function lora_forward\(layer::LoRALinear\{<:DevQ\}, x::ROCArray\{T\}",
    r"function lora_backward\(layer::LoRALinear\{<:DevQ\}, x::ROCArray\{T\}",
    r"ChainRulesCore\.rrule\(::typeof\(lora_forward\), layer::LoRALinear\{<:DevQ\}",
    r"function quantize_frozen_matrix\(w::ROCMatrix\{T\}",
])
def test_seam_methods_exist_for_every_element_type(seam):
    code = " ".join(julia_code().split())
    # the signature itself (within a few lines) constrains T to the three element types
    m = re.search(seam + r"[^\n]{0,200}?where \{?T<:HipFloat", code)
    assert m, f"no method matching {seam} over HipFloat"
    assert "const HipFloat = Union{BFloat16,Float16,Float32}" in code


def test_forward_semantics_follow_the_reference():
    """enabled / active_bias (lora.jl:64-68), dropout refused, alpha / r in Float32."""
    code = " ".join(julia_code().split())
    assert ("_active_bias(layer) = layer.train_bias && !layer.enabled ? layer.base_bias : "
            "layer.bias") in code
    assert "Float32(layer.alpha / size(layer.A, 1))" in code
    assert "layer.enabled && training && layer.dropout > 0" in code
    # the disabled adapter runs the base only (r = 0) with the active bias
    assert "_forward(layer.weight, xf, nothing, nothing, _active_bias(layer), 0f0, false)" in code
