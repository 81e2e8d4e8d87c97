"""crates/ullm-hip cannot be compiled here (no cargo), so its FFI layer is
checked against the C header by text: every entry point include/ullm_hip.h
declares has exactly one `pub fn` in crates/ullm-hip/src/ffi.rs with the same
number of arguments, and the status / dtype constants agree."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _strip_comments(src, c_style=True):
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.sub(r"//[^\n]*", "", src)


def _c_decls():
    src = _strip_comments(open(os.path.join(ROOT, "include", "ullm_hip.h")).read())
    out = {}
    for m in re.finditer(r"\b(ullm_hip_\w+)\s*\(([^;{]*?)\)\s*;", src):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def _rust_decls():
    src = _strip_comments(open(os.path.join(ROOT, "crates", "ullm-hip", "src", "ffi.rs")).read())
    out = {}
    for m in re.finditer(r"pub fn (ullm_hip_\w+)\s*\((.*?)\)\s*(->|;)", src, flags=re.S):
        args = m.group(2).strip().rstrip(",")
        assert m.group(1) not in out, f"{m.group(1)} declared twice"
        out[m.group(1)] = 0 if not args else args.count(":")
    return out


def test_ffi_declares_every_entry_point_with_its_arity():
    c, r = _c_decls(), _rust_decls()
    assert len(c) >= 15
    assert set(c) == set(r), (set(c) ^ set(r))
    for name, n in c.items():
        assert r[name] == n, f"{name}: {r[name]} args in ffi.rs, {n} in the header"


def test_constants_match_the_header():
    h = open(os.path.join(ROOT, "include", "ullm_hip.h")).read()
    rs = open(os.path.join(ROOT, "crates", "ullm-hip", "src", "ffi.rs")).read()
    for name in ("ULLM_HIP_OK", "ULLM_HIP_E_INVALID", "ULLM_HIP_E_UNSUPPORTED", "ULLM_HIP_E_HIP",
                 "ULLM_HIP_E_WORKSPACE", "ULLM_DT_F32", "ULLM_DT_F16", "ULLM_DT_BF16"):
        cv = int(re.search(rf"\b{name}\s*=\s*(-?\d+)", h).group(1))
        rv = int(re.search(rf"pub const {name}: c_int = (-?\d+);", rs).group(1))
        assert cv == rv, name


def _fn_body(src, name):
    i = src.index(f"pub fn {name}(")
    j = src.index("{", src.index(")", i))
    depth, k = 0, j
    while True:
        depth += {"{": 1, "}": -1}.get(src[k], 0)
        k += 1
        if depth == 0:
            return src[j:k]


def test_device_path_neither_copies_nor_waits():
    """forward_dev / forward_batch_dev queue launches only: no host copy and
    no synchronisation inside them (the caller waits once per token), and
    the surface GpuForward has (forward_debug included) is there."""
    src = _strip_comments(open(os.path.join(ROOT, "crates", "ullm-hip", "src", "lib.rs")).read())
    for name in ("forward_dev", "forward_batch_dev"):
        body = _fn_body(src, name)
        for banned in ("hipMemcpy", "upload", "download", "synchronize", "stage("):
            assert banned not in body, f"{name} calls {banned}"
    for name in ("new", "forward", "forward_batch", "supports_batched_prefill", "forward_debug",
                 "synchronize"):
        assert f"pub fn {name}(" in src, name
    # the host-slice wrappers check the slice lengths before any upload
    for name in ("forward", "forward_batch", "forward_debug"):
        body = _fn_body(src, name)
        assert "q.len()" in body or "qs.len()" in body, name
