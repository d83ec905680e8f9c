"""The Zig drop-in (llama.zig_amd/zig/sampler_hip.zig) against the reference's
public sampler API (src/sampler.zig:4-41) and the C ABI it binds.

No Zig toolchain exists here, so the file is checked as text: its public
declarations must equal the reference's (so main.zig:518,667 and
engine.zig:215,355 compile unchanged after the import line), its extern
struct must lay out llz_sampler_config's fields in the C header's order,
and every extern function it declares must be declared by the header and
exported by libllzsample.so.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIM = os.path.join(ROOT, "llama.zig_amd", "zig", "sampler_hip.zig")
HEADER = os.path.join(ROOT, "include", "llz_sampler.h")
LIB = os.path.join(ROOT, "llama.zig_amd", "libllzsample.so")
REF = "/root/reference/src/sampler.zig"

# The reference's public API (sampler.zig:4-41), normalised: whitespace
# collapsed, parameter names kept (Zig call sites may use them positionally
# only, but the text must read the same).
EXPECTED_CONFIG = [
    ("temperature", "f32", "0.8"), ("top_k", "u32", "0"), ("top_p", "f32", "0.9"),
    ("min_p", "f32", "0.0"), ("typical_p", "f32", "1.0"), ("seed", "u64", "0"),
    ("repetition_window", "u32", "32"), ("repetition_penalty", "f32", "1.1"),
]
EXPECTED_FNS = {
    ("Sampler", "init"): "(cfg: SamplerConfig) Sampler",
    ("Sampler", "sample"): "(self: *Sampler, allocator: std.mem.Allocator, logits: []const f32, "
                           "prev_tokens: []const tokenizer.TokenID) !tokenizer.TokenID",
    ("", "sampleArgmax"): "(logits: []const f32) tokenizer.TokenID",
}


def _strip_comments(src: str) -> str:
    return re.sub(r"//[^\n]*", "", src)


def _block(src: str, start: int) -> str:
    """The text of the brace block opening at or after `start`."""
    i = src.index("{", start)
    depth = 0
    for j in range(i, len(src)):
        if src[j] == "{":
            depth += 1
        elif src[j] == "}":
            depth -= 1
            if depth == 0:
                return src[i + 1:j]
    raise ValueError("unbalanced braces")


def _config_fields(src: str):
    m = re.search(r"pub const SamplerConfig = struct", src)
    body = _block(src, m.end())
    return [tuple(f) for f in re.findall(r"(\w+)\s*:\s*([\w\[\]\*]+)\s*=\s*([^,]+),", body)]


def _pub_fns(src: str):
    """{(container, name): normalised signature} of every `pub fn`."""
    out = {}
    sampler_at = re.search(r"pub const Sampler = struct", src)
    sampler_body = _block(src, sampler_at.end())
    body_start = src.index(sampler_body)
    for m in re.finditer(r"pub fn (\w+)\s*(\(.*?\))\s*([^{]+)\{", src, re.S):
        inside = body_start <= m.start() < body_start + len(sampler_body)
        sig = re.sub(r"\s+", " ", m.group(2) + " " + m.group(3)).strip()
        sig = sig.replace("( ", "(").replace(" )", ")").replace(", )", ")")
        out[("Sampler" if inside else "", m.group(1))] = sig
    return out


def _shim():
    with open(SHIM) as f:
        return _strip_comments(f.read())


def test_shim_config_matches_reference_fields_and_defaults():
    assert _config_fields(_shim()) == EXPECTED_CONFIG


def test_shim_public_functions_match_reference_signatures():
    fns = _pub_fns(_shim())
    for key, sig in EXPECTED_FNS.items():
        assert fns.get(key) == sig, (key, fns.get(key))
    # init stays infallible: no error union in its return type
    assert "!" not in fns[("Sampler", "init")]
    # what the shim adds beyond the reference is one optional method
    assert set(fns) - set(EXPECTED_FNS) == {("Sampler", "deinit")}


@pytest.mark.skipif(not os.path.exists(REF), reason="reference checkout not present")
def test_expectations_are_the_reference_declarations():
    """The table above is the reference's own text (read where it exists)."""
    with open(REF) as f:
        ref = _strip_comments(f.read())
    assert _config_fields(ref) == EXPECTED_CONFIG
    ref_fns = _pub_fns(ref)
    assert ref_fns == EXPECTED_FNS


def _header_config_fields():
    with open(HEADER) as f:
        h = f.read()
    body = re.search(r"typedef struct llz_sampler_config \{(.*?)\} llz_sampler_config;", h, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    return re.findall(r"(float|uint32_t|uint64_t)\s+(\w+);", body)


def test_extern_config_layout_matches_header():
    src = _shim()
    m = re.search(r"pub const Config = extern struct", src)
    fields = re.findall(r"(\w+)\s*:\s*(f32|u32|u64)", _block(src, m.end()))
    ctype = {"f32": "float", "u32": "uint32_t", "u64": "uint64_t"}
    assert [(ctype[t], n) for n, t in fields] == _header_config_fields()
    # SamplerConfig's fields appear in the extern struct in the same order
    assert [n for n, _ in fields if n != "reserved"] == [f[0] for f in EXPECTED_CONFIG]


def test_extern_functions_are_declared_and_exported():
    src = _shim()
    names = re.findall(r'pub extern "llzsample" fn (\w+)', src)
    assert names, "the shim binds no C functions"
    with open(HEADER) as f:
        h = f.read()
    for n in names:
        assert re.search(rf"\b{n}\s*\(", h), f"{n} is not declared in include/llz_sampler.h"
    if not os.path.exists(LIB):
        pytest.skip("libllzsample.so not built")
    syms = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in syms.splitlines() if line.strip()}
    for n in names:
        assert n in exported, f"{n} is not exported by libllzsample.so"
