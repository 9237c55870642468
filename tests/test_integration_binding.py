"""The reference-side Rust binding published with this library (the ``hip_ring.rs`` block
of its integration notes, read from the repository root) stays locked to the C ABI.

The reference binds native code through an ``extern "C"`` block
(rust/src/smoke/bridges/cxx.rs:8-70).  The integration notes give the block a maintainer
adds for this library; it cannot be compiled here (no cargo), so this test parses it and
checks it against ``include/hcp_ring.h`` -- every ``#[repr(C)]`` struct field and every
``extern "C"`` function parameter, by name, order and type -- and checks the ctypes
mirrors of the Python package against the header's struct layouts.  A field dropped,
added, reordered or retyped on either side fails it (the last tests plant such
mistakes and require the comparison to catch them).
"""
import ctypes
import os
import re

import pytest

import hcp_ring_amd as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hcp_ring.h")
INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")

C_SCALARS = {"int32_t": "i32", "int64_t": "i64", "uint64_t": "u64", "uint32_t": "u32", "uint8_t": "u8",
             "float": "f32", "double": "f64", "int": "c_int", "size_t": "usize", "char": "c_char",
             "void": "c_void"}
C_SIZES = {"int32_t": 4, "int64_t": 8, "uint64_t": 8, "uint32_t": 4, "uint8_t": 1, "float": 4, "double": 8,
           "int": 4, "size_t": 8, "char": 1}


def camel(name: str) -> str:
    return "".join(p.capitalize() for p in name.split("_"))


def c_to_rust(ctype: str) -> str:
    """The Rust spelling of a C parameter / field type: `const T*` -> `*const T`,
    `T*` -> `*mut T`, a `const` after a `*` makes the next pointer level const."""
    m = re.match(r"^(const\s+)?(\w+)\s*((?:\*\s*(?:const\s*)?)*)$", ctype.strip())
    assert m, ctype
    base = C_SCALARS.get(m.group(2)) or camel(m.group(2))
    levels = re.findall(r"\*\s*(const)?", m.group(3))
    quals = ([bool(m.group(1))] + [bool(x) for x in levels[:-1]]) if levels else []
    for const in quals:
        base = ("*const " if const else "*mut ") + base
    return base


def strip_c_comments(text: str) -> str:
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))


def parse_header(text: str):
    text = strip_c_comments(text)
    structs = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} \w+;", text, re.S):
        fields = []
        for f in (x.strip() for x in m.group(2).split(";")):
            if not f:
                continue
            a = re.match(r"^(.*?)(\w+)\s*(?:\[(\w+)\])?$", f)
            fields.append((a.group(2), a.group(1).strip(), a.group(3)))
        structs[m.group(1)] = fields
    fns = {}
    for m in re.finditer(r"^\s*([a-z_0-9 ]+\**)\s+(\**)(hcp_[a-z_0-9]+)\s*\((.*?)\);", text, re.S | re.M):
        args = " ".join(m.group(4).split())
        params = []
        if args != "void":
            for a in args.split(","):
                am = re.match(r"^(.*?)(\w+)$", a.strip())
                params.append((am.group(2), am.group(1).strip()))
        fns[m.group(3)] = ((m.group(1) + m.group(2)).strip(), params)
    defines = dict(re.findall(r"#define (\w+) (\S+)", text))
    return structs, fns, defines


def rust_block(md: str) -> str:
    m = re.search(r"```rust\n(// rust/src/model/attention/hip_ring\.rs.*?)```", md, re.S)
    assert m, "INTEGRATION.md has no hip_ring.rs block"
    return m.group(1)


def parse_rust(block: str):
    body = re.sub(r"//[^\n]*", "", block)
    structs = {}
    for m in re.finditer(r"#\[repr\(C\)\](?:\s*#\[derive\([^)]*\)\])?\s*pub struct (\w+)\s*\{(.*?)\}", body, re.S):
        fields = []
        for f in (x.strip() for x in m.group(2).split(",")):
            if not f:
                continue
            fm = re.match(r"^(pub\s+)?(\w+)\s*:\s*(.+)$", f)
            fields.append((fm.group(2), " ".join(fm.group(3).split())))
        structs[m.group(1)] = fields
    ext = re.search(r'extern "C" \{(.*?)\n\}', body, re.S).group(1)
    fns = {}
    order = []
    for m in re.finditer(r"pub fn (\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", ext, re.S):
        params = []
        args = " ".join(m.group(2).split())
        if args:
            for a in args.split(","):
                if not a.strip():
                    continue
                name, ty = a.split(":", 1)
                params.append((name.strip(), " ".join(ty.split())))
        fns[m.group(1)] = ((m.group(3) or "").strip(), params)
        order.append(m.group(1))
    consts = dict(re.findall(r"pub const (\w+)\s*:\s*\w+\s*=\s*(\d+)\s*;", body))
    return structs, fns, consts, order


def compare(hdr_structs, hdr_fns, rs_structs, rs_fns):
    """Differences between the header and the Rust block, as readable strings."""
    errs = []
    opaque = {n for n, f in rs_structs.items() if [x[0] for x in f] == ["_opaque"]}
    want_structs = {camel(n): n for n in hdr_structs}
    for name in sorted(set(want_structs) ^ (set(rs_structs) - opaque)):
        errs.append(f"struct {name} on one side only")
    for rname, cname in want_structs.items():
        if rname not in rs_structs:
            continue
        want = [(f, c_to_rust(t) if n is None else f"[{c_to_rust(t)}; {n}]") for f, t, n in hdr_structs[cname]]
        if rs_structs[rname] != want:
            errs.append(f"struct {rname}: rust {rs_structs[rname]} != header {want}")
    for name in sorted(set(hdr_fns) ^ set(rs_fns)):
        errs.append(f"function {name} on one side only")
    for name, (ret, params) in hdr_fns.items():
        if name not in rs_fns:
            continue
        want_ret = "" if ret == "void" else c_to_rust(ret)
        want = [(p, c_to_rust(t)) for p, t in params]
        if rs_fns[name] != (want_ret, want):
            errs.append(f"fn {name}: rust {rs_fns[name]} != header {(want_ret, want)}")
    return errs


@pytest.fixture(scope="module")
def sides():
    hdr = parse_header(open(HEADER).read())
    rs = parse_rust(rust_block(open(INTEGRATION).read()))
    return hdr, rs


def test_rust_binding_matches_header(sides):
    (hs, hf, hd), (rs, rf, rc, order) = sides
    assert len(hs) >= 13 and len(hf) >= 55
    assert compare(hs, hf, rs, rf) == []
    # in header order, so a reader can follow both side by side
    assert order == [n for n in re.findall(r"(hcp_[a-z_0-9]+)\s*\(", strip_c_comments(open(HEADER).read()))
                     if n in hf and n in order][:len(order)]


def test_rust_binding_constants_and_abi_check(sides):
    (hs, hf, hd), (rs, rf, rc, order) = sides
    assert int(rc["HCP_RING_ABI_VERSION"]) == int(hd["HCP_RING_ABI_VERSION"]) == H.ABI_VERSION
    assert int(rc["HCP_BLOCK_AGENT_MAX"]) == int(hd["HCP_BLOCK_AGENT_MAX"])
    assert int(rc["HCP_BLOCK_META_MAX"]) == int(hd["HCP_BLOCK_META_MAX"])
    block = rust_block(open(INTEGRATION).read())
    assert "pub fn hcp_ring_check_abi()" in block and "hcp_ring_abi_version()" in block
    # the replay descriptor carries the schedule the library validates (ABI >= 2)
    assert [f for f, _ in rs["HcpRingReplayDesc"]][-2:] == ["strategy", "schedule"]


def _c_layout(fields, structs):
    """(size, align, offsets) of a C struct with natural alignment (x86-64 / amdgcn)."""
    off, align, offs = 0, 1, []
    for name, ctype, n in fields:
        t = ctype.replace("const", "").strip()
        if "*" in t:
            size = al = 8
        elif t in C_SIZES:
            size = al = C_SIZES[t]
        else:
            size, al, _ = _c_layout(structs[t], structs)
        count = 1
        if n is not None:
            count = {"HCP_BLOCK_META_MAX": 256, "HCP_BLOCK_AGENT_MAX": 64}.get(n) or int(n)
        off = (off + al - 1) // al * al
        offs.append((name, off))
        off += size * count
        align = max(align, al)
    return (off + align - 1) // align * align, align, offs


CTYPES_MIRRORS = {
    "View": "hcp_ring_view", "BlockDesc": "hcp_ring_block_desc", "PagedPool": "hcp_paged_pool",
    "PagedRange": "hcp_paged_range", "DecodeShard": "hcp_decode_shard", "DecodeDesc": "hcp_paged_decode_desc",
    "ReplayDesc": "hcp_ring_replay_desc", "BlockDescC": "hcp_block_desc",
    "RemoteBlockDescC": "hcp_remote_block_desc", "BlockCompletionC": "hcp_block_completion",
    "KvFrameDesc": "hcp_kv_frame_desc", "PacketFrameDesc": "hcp_packet_frame_desc", "QkvDesc": "hcp_qkv_desc",
    "TraceDomain": "hcp_ring_trace_domain", "TraceLaunch": "hcp_ring_trace_launch",
}


def test_ctypes_mirrors_match_header_layouts(sides):
    (hs, hf, hd), _ = sides
    assert set(CTYPES_MIRRORS.values()) == set(hs)
    for cls_name, cname in CTYPES_MIRRORS.items():
        cls = getattr(H, cls_name)
        size, _, offs = _c_layout(hs[cname], hs)
        assert [f[0] for f in cls._fields_] == [f[0] for f in hs[cname]], cls_name
        assert ctypes.sizeof(cls) == size, cls_name
        assert [(n, getattr(cls, n).offset) for n, _ in offs] == offs, cls_name


def test_comparison_catches_planted_drift(sides):
    # a dropped field on either side, a reordered field, a retyped parameter and a
    # missing function are all reported
    (hs, hf, hd), (rs, rf, rc, order) = sides
    rs1 = {k: list(v) for k, v in rs.items()}
    rs1["HcpRingReplayDesc"] = rs1["HcpRingReplayDesc"][:-1]  # the stale v1 binding
    assert any("HcpRingReplayDesc" in e for e in compare(hs, hf, rs1, rf))
    hs1 = {k: list(v) for k, v in hs.items()}
    hs1["hcp_ring_block_desc"] = hs1["hcp_ring_block_desc"][:-1]
    assert any("HcpRingBlockDesc" in e for e in compare(hs1, hf, rs, rf))
    rs2 = {k: list(v) for k, v in rs.items()}
    f = rs2["HcpPagedPool"]
    f[2], f[3] = f[3], f[2]
    assert any("HcpPagedPool" in e for e in compare(hs, hf, rs2, rf))
    rf1 = dict(rf)
    ret, params = rf1["hcp_ring_block_partial"]
    rf1["hcp_ring_block_partial"] = (ret, [(n, "*mut f64" if n == "o" else t) for n, t in params])
    assert any("hcp_ring_block_partial" in e for e in compare(hs, hf, rs, rf1))
    rf2 = {k: v for k, v in rf.items() if k != "hcp_ring_prefill_replay_paged"}
    assert any("hcp_ring_prefill_replay_paged" in e for e in compare(hs, hf, rs, rf2))


def test_ctypes_comparison_catches_planted_drift(sides):
    (hs, hf, hd), _ = sides

    class Stale(ctypes.Structure):  # ReplayDesc without schedule
        _fields_ = H.ReplayDesc._fields_[:-1]

    size, _, offs = _c_layout(hs["hcp_ring_replay_desc"], hs)
    assert ctypes.sizeof(Stale) != size or [f[0] for f in Stale._fields_] != [n for n, _ in offs]
