"""Source-text checks of integration/backend_hip.zig against the C ABI (no Zig
toolchain exists here or on the GPU box, so the file is checked as text, the
way the reference checks its CUDA seam in src/backend_cuda_launch_tests.zig:
92-163): every `extern fn qhip_*` it declares is declared in
include/qwen35_hip.h with the same number of parameters and compatible
types and is exported by the library; its `QhipLinear` is the header's
`qhip_linear`; it calls no `qhip_launch_*` kernel entry directly (the backend
slots are the seam); and the slots it replaces are exactly the quantized-matvec
slots of the reference's Exec vtable (src/backend.zig:110-178)."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ZIG = ROOT / "integration" / "backend_hip.zig"
HEADER = ROOT / "include" / "qwen35_hip.h"
REF_BACKEND = Path("/root/reference/src/backend.zig")

# the Exec slots of the quantized-matvec path and its support slots
# (src/backend.zig:110-178, :470-514)
MATVEC_SLOTS = {"loadLinear", "freeLinear", "matvec", "matvecPair", "matvecBatchK", "dequantRow",
                "allocScratch", "allocScratchK", "freeScratch", "allocBuf", "stepBegin", "stepEnd", "name",
                "describe", "reportProfile", "profReport"}

# Zig parameter / return type -> the C type it must be
ZIG_TO_C = {"c_int": "int", "c_long": "long", "c_uint": "unsigned", "usize": "size_t", "void": "void",
            "f32": "float"}


def strip_zig_comments(text):
    return "\n".join(l.split("//")[0] for l in text.splitlines())


def zig_externs():
    text = strip_zig_comments(ZIG.read_text())
    out = {}
    for m in re.finditer(r"extern fn (\w+)\((.*?)\)\s*([^;]+);", text, flags=re.S):
        name, params, ret = m.group(1), m.group(2), m.group(3).strip()
        ps = [p.strip() for p in params.split(",") if p.strip()]
        out[name] = ([p.split(":", 1)[1].strip() for p in ps], ret)
    return out


def c_decls():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(qhip_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        ps = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        out[name] = (ps, ret)
    return out


def c_type(decl):
    """'const float *d_x' -> 'ptr'; 'int rows' -> 'int'; 'size_t bytes' -> 'size_t'."""
    if "*" in decl:
        return "ptr"
    words = decl.replace("const", "").split()
    return " ".join(words[:-1]) if len(words) > 1 else words[0]


def z_type(t):
    t = t.strip()
    if t.startswith(("?", "*", "[")):
        return "ptr"
    return ZIG_TO_C.get(t, t)


def test_externs_match_the_header():
    ext = {n: v for n, v in zig_externs().items() if n.startswith("qhip_")}
    decl = c_decls()
    assert len(ext) >= 15
    for name, (zp, zr) in ext.items():
        assert name in decl, f"{name} is not declared in include/qwen35_hip.h"
        cp, cr = decl[name]
        assert len(zp) == len(cp), (name, zp, cp)
        for z, c in zip(zp, cp):
            assert z_type(z) == c_type(c), (name, z, c)
        cret = "ptr" if "*" in cr else cr.replace("const", "").strip()
        assert z_type(zr) == cret, (name, zr, cr)


def test_other_externs_are_the_hip_runtime_host_allocator():
    other = sorted(n for n in zig_externs() if not n.startswith("qhip_"))
    assert other == ["hipHostFree", "hipHostMalloc"]


def test_externs_are_exported_by_the_library():
    so = ROOT / "qwen35_amd" / "libqwen35_hip.so"
    if not so.exists():
        pytest.skip("library not built")
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (qhip_\w+)", out))
    missing = [n for n in zig_externs() if n.startswith("qhip_") and n not in exported]
    assert not missing, missing


def test_linear_struct_matches_the_header():
    text = strip_zig_comments(ZIG.read_text())
    zs = re.search(r"const QhipLinear = extern struct \{(.*?)\};", text, flags=re.S).group(1)
    zf = [(f.split(":")[0].strip(), z_type(f.split(":")[1])) for f in zs.split(",") if f.strip()]
    hs = re.search(r"typedef struct qhip_linear \{(.*?)\} qhip_linear;",
                   re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S), flags=re.S).group(1)
    hf = [(d.split()[-1].lstrip("*"), c_type(d)) for d in (x.strip() for x in hs.split(";")) if d]
    assert zf == hf


def test_no_kernel_entry_bypasses_the_backend_seam():
    # qhip_launch_* are the kernel-level entry points; the Zig backend must
    # reach the device only through the qhip_backend_* slots
    code = strip_zig_comments(ZIG.read_text())
    assert "qhip_launch_" not in code


def test_replaced_slots_are_the_matvec_path():
    text = strip_zig_comments(ZIG.read_text())
    body = re.search(r"pub const vtable: backend\.Exec\.VTable = blk: \{(.*?)break :blk vt;", text, flags=re.S)
    assert body, "vtable block not found"
    replaced = set(re.findall(r"vt\.(\w+) = \w+;", body.group(1)))
    assert replaced == MATVEC_SLOTS
    if REF_BACKEND.exists():  # the slot names exist in the reference's vtable
        ref = REF_BACKEND.read_text()
        for slot in replaced:
            assert re.search(rf"\b{slot}: \*const fn", ref), slot


def test_every_slot_function_is_defined():
    text = strip_zig_comments(ZIG.read_text())
    body = re.search(r"pub const vtable: backend\.Exec\.VTable = blk: \{(.*?)break :blk vt;", text, flags=re.S)
    for fn in re.findall(r"vt\.\w+ = (\w+);", body.group(1)):
        assert re.search(rf"\bfn {fn}\(", text), fn
