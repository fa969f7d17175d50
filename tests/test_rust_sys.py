"""The Rust -sys crate (h3-hrx_amd/h3attn-sys) against include/h3attn.h. No Rust toolchain is in
this image, so the crate cannot be compiled here; these checks keep its source in step with the
header it binds: every function the header declares has an `extern "C"` declaration with the
same parameter count, every struct mirror has the header's fields in the header's order, and the
crate's layout test expects the sizes the ctypes binding (and so the C compiler) gives."""
import ctypes
import pathlib
import re
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "h3-hrx_amd"))

import h3attn as H  # noqa: E402

HEADER = (ROOT / "include" / "h3attn.h").read_text()
LIB_RS = (ROOT / "h3-hrx_amd" / "h3attn-sys" / "src" / "lib.rs").read_text()


def strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def header_functions():
    body = strip_c_comments(HEADER)
    out = {}
    for m in re.finditer(r"\b(h3_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", body):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def rust_functions():
    out = {}
    for m in re.finditer(r"pub fn (h3_[a-z0-9_]+)\s*\(([^)]*)\)", LIB_RS):
        params = m.group(2).strip().rstrip(",")
        out[m.group(1)] = 0 if not params else params.count(",") + 1
    return out


def test_every_header_function_is_declared_with_its_arity():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 50
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, n in h.items():
        assert r[name] == n, (name, n, r[name])


def header_struct_fields(name):
    body = strip_c_comments(HEADER)
    m = re.search(r"typedef struct \{([^}]*)\}\s*" + name + r"\s*;", body)
    assert m, name
    fields = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split(None, 1)[1] if not decl.startswith("const ") else decl.rsplit(None, 1)[1]
        for f in names.replace("*", " ").split(","):
            fields.append(f.strip().split()[-1])
    return fields


def rust_struct_fields(name):
    m = re.search(r"pub struct " + name + r"\s*\{([^}]*)\}", LIB_RS)
    assert m, name
    return re.findall(r"pub (\w+):", m.group(1))


PAIRS = [("h3_prepare_cfg", "H3PrepareCfg"), ("h3_rope_cfg", "H3RopeCfg"),
         ("h3_transpose_cfg", "H3TransposeCfg"), ("h3_gemm_cfg", "H3GemmCfg"),
         ("h3_prepare_plain_cfg", "H3PreparePlainCfg"), ("h3_attention_cfg", "H3AttentionCfg"),
         ("h3_attention_skip_cfg", "H3AttentionSkipCfg"), ("h3_cross_cfg", "H3CrossCfg"),
         ("h3_vsa_cfg", "H3VsaCfg"), ("h3_vsa_segment", "H3VsaSegment"),
         ("h3_vsa_options", "H3VsaOptions"), ("h3_stack_dims", "H3StackDims"),
         ("h3_vsa_buffers", "H3VsaBuffers"), ("h3_int_qk", "H3IntQk"), ("h3_view", "H3View")]


def test_struct_mirrors_have_the_header_fields_in_order():
    for c_name, rs_name in PAIRS:
        assert header_struct_fields(c_name) == rust_struct_fields(rs_name), c_name


def test_layout_test_sizes_match_the_c_layouts():
    sizes = dict(re.findall(r"size_of::<(\w+)>\(\), (\d+)\)", LIB_RS))
    py = {"H3View": H.View, "H3PrepareCfg": H.PrepareCfg, "H3RopeCfg": H.RopeCfg,
          "H3TransposeCfg": H.TransposeCfg, "H3GemmCfg": H.GemmCfg,
          "H3PreparePlainCfg": H.PreparePlainCfg, "H3AttentionCfg": H.AttentionCfg,
          "H3AttentionSkipCfg": H.AttentionSkipCfg, "H3CrossCfg": H.CrossCfg,
          "H3VsaCfg": H.VsaCfg, "H3StackDims": H.StackDims}
    assert set(sizes) == set(py)
    for k, cls in py.items():
        assert int(sizes[k]) == ctypes.sizeof(cls), k


def test_capacity_examples_match_the_library():
    for t, want in re.findall(r"h3_capacity\(([\d_]+), 0\) \}, ([\d_]+)\)", LIB_RS):
        assert H.capacity(int(t.replace("_", ""))) == int(want.replace("_", ""))


def test_manifest_links_the_library():
    cargo = (ROOT / "h3-hrx_amd" / "h3attn-sys" / "Cargo.toml").read_text()
    build = (ROOT / "h3-hrx_amd" / "h3attn-sys" / "build.rs").read_text()
    assert 'links = "h3attn"' in cargo
    assert "rustc-link-lib=dylib=h3attn" in build
