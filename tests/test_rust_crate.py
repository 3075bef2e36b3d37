"""The Rust binding crate (crates/vllm-hip, source only: no Rust toolchain in this image) agrees
with the C ABI and with Railgun's launcher API.

* ffi.rs declares exactly the functions of include/railgun_hip.h, each with the same
  parameter names, the Rust type that matches each C type, and the matching return type;
* kernels.rs has every launcher of PagedAttentionKernels
  (crates/vllm-cuda/src/kernels/mod.rs:196-508) with the same parameter names in the same
  order, and op.rs the methods of PagedAttentionOp (paged_attn_op.rs:45-268).
"""
from __future__ import annotations

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "railgun_hip.h")
CRATE = os.path.join(ROOT, "crates", "vllm-hip", "src")

C_TO_RUST = {
    "const void*": "*const c_void", "void*": "*mut c_void", "const int32_t*": "*const i32", "int32_t*": "*mut i32",
    "const float*": "*const f32", "float*": "*mut f32", "int32_t": "i32", "int64_t": "i64", "size_t": "usize",
    "float": "f32", "double": "f64", "int": "c_int", "const char*": "*const c_char",
}

# Launchers of mod.rs:196-508, parameter names in order (after &self).
MOD_RS_LAUNCHERS = {
    "launch_rope": ["x", "cos_sin", "positions", "num_heads", "head_dim", "num_tokens"],
    "launch_reshape_and_cache": ["k", "v", "k_cache", "v_cache", "slot_mapping", "num_kv_heads", "head_dim",
                                 "block_size", "batch_size"],
    "launch_reshape_and_cache_isoquant": ["k", "v", "k_cache", "v_cache", "slot_mapping", "rotation_metadata",
                                          "num_kv_heads", "head_dim", "block_size", "batch_size"],
    "launch_v1": ["query", "key_cache", "value_cache", "block_table", "context_lens", "output", "scale",
                  "num_heads", "num_kv_heads", "head_dim", "block_size", "max_blocks_per_seq", "batch_size"],
    "launch_v1_plus": ["query", "key_cache", "value_cache", "block_table", "context_lens", "output",
                       "rotation_metadata", "scale", "num_heads", "num_kv_heads", "head_dim", "block_size",
                       "max_blocks_per_seq", "batch_size"],
    "launch_v2_partition": ["query", "key_cache", "value_cache", "block_table", "context_lens", "tmp_out",
                            "exp_sums", "max_logits", "rotation_metadata", "scale", "num_heads", "num_kv_heads",
                            "head_dim", "block_size", "max_blocks_per_seq", "num_partitions", "batch_size"],
    "launch_v2_reduce": ["output", "exp_sums", "max_logits", "tmp_out", "context_lens", "rotation_metadata",
                         "num_heads", "head_dim", "num_partitions", "batch_size"],
}
# PagedAttentionOp (paged_attn_op.rs:45-54, 168-177, 236-241).
OP_METHODS = {
    "execute": ["q", "k_cache", "v_cache", "block_table", "context_lens", "rotation_metadata", "max_context_len"],
    "reshape_and_cache": ["k", "v", "k_cache", "v_cache", "slot_mapping", "rotation_metadata", "use_isoquant"],
    "apply_rope": ["x", "cos_sin", "positions"],
}


def _norm_c(t: str) -> str:
    return re.sub(r"\s*\*", "*", re.sub(r"\s+", " ", t.strip()))


def header_prototypes() -> dict[str, tuple[str, list[tuple[str, str]]]]:
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"^((?:const\s+)?[a-z_0-9]+\s*\*?)\s*(rg_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;",
                                      text, re.M | re.S):
        params = []
        if args.strip() not in ("", "void"):
            for a in args.split(","):
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", a.strip())
                params.append((m.group(2), _norm_c(m.group(1))))
        out[name] = (_norm_c(ret), params)
    return out


def _split_params(text: str) -> list[str]:
    """Top-level comma split (generic brackets may hold commas)."""
    parts, depth, cur = [], 0, ""
    for ch in text:
        if ch in "<([":
            depth += 1
        elif ch in ">)]":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur)
    return [p.strip() for p in parts if p.strip()]


def rust_fns(path: str) -> dict[str, tuple[str, list[tuple[str, str]]]]:
    """fn name -> (return type, [(param, type)]) for every `fn` in a Rust file (self excluded)."""
    text = re.sub(r"//[^\n]*", "", open(path).read())
    out = {}
    for m in re.finditer(r"\bfn\s+([A-Za-z_0-9]+)\s*(?:<[^>]*>)?\s*\((.*?)\)\s*(?:->\s*([^;{]+?))?\s*[;{]", text,
                         re.S):
        params = []
        for p in _split_params(m.group(2)):
            if p.lstrip("&").startswith("mut self") or p.lstrip("&").startswith("self"):
                continue
            name, typ = p.split(":", 1)
            params.append((name.strip().removeprefix("mut "), re.sub(r"\s+", " ", typ.strip())))
        out[m.group(1)] = ((m.group(3) or "()").strip(), params)
    return out


def ffi_mismatches(r: dict) -> list[str]:
    """Differences between the header's prototypes and parsed Rust declarations."""
    c = header_prototypes()
    errs = []
    if set(r) != set(c):
        errs.append(f"only in header: {set(c) - set(r)}; only in ffi.rs: {set(r) - set(c)}")
    for name, (ret, params) in c.items():
        if name not in r:
            continue
        rret, rparams = r[name]
        if rret != C_TO_RUST[ret]:
            errs.append(f"{name}: returns {rret}, header {ret}")
        if len(rparams) != len(params):
            errs.append(f"{name}: {len(rparams)} parameters, header {len(params)}")
        for (cn, ct), (rn, rt) in zip(params, rparams):
            if rn != cn:
                errs.append(f"{name}: parameter {rn} where the header has {cn}")
            if rt != C_TO_RUST[ct]:
                errs.append(f"{name}({cn}): {rt} for C {ct}")
    return errs


def test_ffi_matches_header():
    assert len(header_prototypes()) >= 21
    assert ffi_mismatches(rust_fns(os.path.join(CRATE, "ffi.rs"))) == []


def test_ffi_check_catches_a_swapped_parameter(tmp_path):
    """The comparison sees a plausible mistake: two adjacent i32 parameters swapped in one
    declaration (the types still agree), and an i64 stride declared as i32."""
    text = open(os.path.join(CRATE, "ffi.rs")).read()
    swapped = text.replace("num_heads: i32, num_kv_heads: i32", "num_kv_heads: i32, num_heads: i32", 1)
    narrowed = text.replace("kv_block_stride: i64", "kv_block_stride: i32", 1)
    for bad in (swapped, narrowed):
        assert bad != text
        f = tmp_path / "ffi.rs"
        f.write_text(bad)
        assert ffi_mismatches(rust_fns(str(f)))


def test_ffi_constants_match_header():
    hdr = open(HEADER).read()
    ffi = open(os.path.join(CRATE, "ffi.rs")).read()
    for name, val in re.findall(r"#define (RG_[A-Z0-9_]+) (\d+)\b", hdr):
        m = re.search(rf"pub const {name}: [a-z_0-9]+ = (\d+);", ffi)
        assert m and m.group(1) == val, f"{name} = {val} in the header"
    m = re.search(r"#define RG_NO_ALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", hdr)
    assert m and f"RG_NO_ALLOC_SCRATCH_BYTES: usize = {m.group(1)} << {m.group(2)};" in ffi


def test_kernels_mirror_reference_launchers():
    r = rust_fns(os.path.join(CRATE, "kernels.rs"))
    for name, params in MOD_RS_LAUNCHERS.items():
        assert name in r, f"kernels.rs lacks {name}"
        assert [p for p, _ in r[name][1]] == params, f"{name}: {[p for p, _ in r[name][1]]}"
        assert r[name][0] == "CoreResult<()>"
    assert "new" in r and r["new"][0] == "CoreResult<Self>"


def test_op_mirrors_reference_methods():
    r = rust_fns(os.path.join(CRATE, "op.rs"))
    for name, params in OP_METHODS.items():
        assert name in r, f"op.rs lacks {name}"
        assert [p for p, _ in r[name][1]] == params, f"{name}: {[p for p, _ in r[name][1]]}"
        assert r[name][0].startswith("CoreResult<")


def test_every_ffi_entry_is_called_by_the_crate():
    """Each C entry has a safe(r) wrapper in kernels.rs (or op.rs) that calls it."""
    body = open(os.path.join(CRATE, "kernels.rs")).read() + open(os.path.join(CRATE, "op.rs")).read()
    for name in header_prototypes():
        assert f"ffi::{name}(" in body, f"no wrapper calls {name}"


def _fn_body(path: str, name: str) -> str:
    """The text of `pub fn name` in a Rust source file, up to the next `pub fn` or the file's end."""
    text = open(path).read()
    m = re.search(rf"pub (?:unsafe )?fn {name}\b", text)
    assert m, f"{name} not found in {path}"
    nxt = re.search(r"\n    pub (?:unsafe )?fn ", text[m.end():])
    return text[m.start():m.end() + (nxt.start() if nxt else len(text))]


# Calls that stall the host or allocate device scratch on every call.
_STALLS = ("hipStreamSynchronize", "hipDeviceSynchronize", "hipEventSynchronize", "hipMalloc", "hipFree",
           "HipSlice::<u8>::alloc")


def test_execute_neither_synchronises_nor_allocates_scratch(tmp_path):
    """PagedAttentionOp::execute queues its launches and returns: the split-K scratch is the
    kernels' grow-only workspace (with_workspace), never a per-call allocation freed after a
    stream synchronisation.  The check is shown to see a synchronize planted in the body."""
    op_rs = os.path.join(CRATE, "op.rs")
    body = _fn_body(op_rs, "execute")
    for call in _STALLS:
        assert call not in body, f"execute calls {call}"
    assert body.count("with_workspace(") == 2, "both branches (v1+, v2) take the shared workspace"
    planted = tmp_path / "op.rs"
    planted.write_text(open(op_rs).read().replace("        Ok(out)\n",
                                                  "        crate::hip::hipStreamSynchronize(k.stream());\n"
                                                  "        Ok(out)\n", 1))
    assert any(call in _fn_body(str(planted), "execute") for call in _STALLS)
    # The workspace lives in the kernels object, which one Arc shares across layers
    # (vllm-models model.rs:127), grows only when a call needs more, and is never freed by execute.
    grow = _fn_body(os.path.join(CRATE, "kernels.rs"), "with_workspace")
    assert "w.len() < bytes" in grow and "HipSlice::<u8>::alloc" in grow


def test_op_fields_match_the_reference_struct():
    """The op keeps exactly the reference's public fields (paged_attn_op.rs:12-19), so the
    struct literal of its call site (vllm-models attention.rs:109-116) builds it unchanged."""
    text = open(os.path.join(CRATE, "op.rs")).read()
    m = re.search(r"pub struct PagedAttentionOp \{(.*?)\n\}", text, re.S)
    assert m
    fields = re.findall(r"^\s*(pub\s+)?([a-z_]+):", m.group(1), re.M)
    assert [(bool(p), n) for p, n in fields] == [(True, n) for n in
                                                 ("scale", "num_heads", "num_kv_heads", "head_dim", "block_size",
                                                  "kernels")]
