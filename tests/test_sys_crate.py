"""The Rust `-sys` crate (crates/ramvamp-attn-sys) cannot drift from the
library: its extern "C" block declares exactly the functions include/*.h
declares, with the same parameter counts and names; its constants match the
header's; and its build.rs compiles the sources, with the flags, that
ramvamp_amd/build.py compiles. (rustc/cargo are not in this image, so the
crate is checked as text here.)"""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "crates", "ramvamp-attn-sys")
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def header_prototypes():
    """name -> parameter names, straight from the C text."""
    protos = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", " ", open(h).read(), flags=re.S)
        text = re.sub(r"typedef\s+(struct|enum)\s+\w+\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
        for m in re.finditer(r"\b(rv_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            params = " ".join(m.group(2).split())
            names = [] if params in ("", "void") else [re.findall(r"\w+", p)[-1] for p in params.split(",")]
            protos[m.group(1)] = names
    return protos


def crate_prototypes():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = text[text.index('extern "C" {'):]
    protos = {}
    for m in re.finditer(r"pub fn (rv_\w+)\((.*?)\)", block, flags=re.S):
        args = " ".join(m.group(2).split())
        protos[m.group(1)] = [] if not args else [a.split(":")[0].strip() for a in args.split(",")]
    return protos


def test_extern_block_matches_the_headers_by_name_and_arity():
    h, c = header_prototypes(), crate_prototypes()
    assert len(h) >= 50
    assert set(h) == set(c), set(h) ^ set(c)
    for name in h:
        assert h[name] == c[name], (name, h[name], c[name])


def test_constants_match_the_headers():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    crate = dict(re.findall(r"pub const (RV_\w+): \w+ = (.+);", text))
    for hpath in HEADERS:
        for name, val in re.findall(r"^#define\s+(RV_[A-Z0-9_]+)\s+(\S+)", open(hpath).read(), flags=re.M):
            if name.endswith("_H") or val.startswith("((size_t)"):
                continue
            assert name in crate, name
            assert int(crate[name], 0) == int(val.rstrip("u"), 0), (name, crate[name], val)


def test_build_rs_compiles_what_build_py_compiles():
    sys.path.insert(0, ROOT)
    from ramvamp_amd import build as B
    text = open(os.path.join(CRATE, "build.rs")).read()
    srcs = re.findall(r'"([\w.]+\.(?:hip|cpp))"', text.split("const FLAGS")[0])
    assert srcs == B.SOURCES
    flags = re.findall(r'"([^"]+)"', re.search(r"const FLAGS: &\[&str\] = &\[(.*?)\];", text).group(1))
    assert flags == B.FLAGS
    for src, extra in B.EXTRA.items():
        m = re.search(r'\("' + re.escape(src) + r'", &\[(.*?)\]\)', text)
        assert m and re.findall(r'"([^"]+)"', m.group(1)) == extra, src


def test_generated_files_are_current():
    rc = subprocess.run([sys.executable, os.path.join(CRATE, "gen_bindings.py"), "--check"], capture_output=True,
                        text=True)
    assert rc.returncode == 0, rc.stderr
