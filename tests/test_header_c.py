"""The boundary header compiles for C and C++ consumers.

include/wpcg.h is what a reference-side binding (a Rust `extern "C"` block,
a C caller) is written against. These tests compile a translation unit that
includes it and calls every declared function with arguments of exactly
the declared parameter types, as C11 and as C++17, with every warning an
error. A struct tag first seen inside a parameter list (prototype scope in
C), a mismatched typedef or a missing declaration fails here. No GPU and no
library call: the unit is compiled, not run.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wpcg.h")


def _prototypes():
    """(return type, name, [parameter types]) of every function the header declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
    protos = []
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(wpcg_[a-z0-9_]+)\s*\(([^;{)]*)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        if ret.startswith("typedef"):
            continue
        types = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                # drop the parameter name (the last identifier)
                t = re.sub(r"\s*\b[A-Za-z_][A-Za-z0-9_]*$", "", p).strip()
                assert t, (name, p)
                types.append(t)
        protos.append((ret, name, types))
    return protos


def _unit():
    lines = ["#include \"wpcg.h\"", "", "int wpcg_header_use_all(void);",
             "int wpcg_header_use_all(void) {", "    int s = 0;"]
    for ret, name, types in _prototypes():
        args = ", ".join(f"({t})0" for t in types)
        call = f"{name}({args})"
        if ret == "int":
            lines.append(f"    s += {call};")
        else:
            lines.append(f"    s += ({call}) != 0;")
    lines += ["    return s;", "}", ""]
    return "\n".join(lines)


def test_every_function_is_parsed():
    names = {n for _, n, _ in _prototypes()}
    declared = set(re.findall(r"\b(wpcg_[a-z0-9_]+)\s*\(",
                              re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)))
    assert names == declared
    assert len(names) >= 60


@pytest.mark.parametrize("lang,compiler,flags", [
    ("c", "gcc", ["-std=c11", "-pedantic"]),
    ("c", "gcc", ["-std=c99", "-pedantic"]),
    ("c++", "g++", ["-std=c++17", "-pedantic"]),
])
def test_header_compiles_with_every_call(tmp_path, lang, compiler, flags):
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    src = tmp_path / ("use_all.c" if lang == "c" else "use_all.cpp")
    src.write_text(_unit())
    cmd = [compiler, *flags, "-Wall", "-Wextra", "-Werror", "-I", os.path.dirname(HEADER),
           "-c", str(src), "-o", str(tmp_path / "use_all.o")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_config_struct_usable_before_and_after_definition(tmp_path):
    """A C caller fills wpcg_model_config and hands it to both the parser and
    wpcg_model_create, the sequence a binding performs."""
    src = tmp_path / "cfg.c"
    src.write_text("""#include "wpcg.h"
int f(const char* json, wpcg_ctx* ctx, wpcg_model** out);
int f(const char* json, wpcg_ctx* ctx, wpcg_model** out) {
    wpcg_model_config cfg;
    int rc = wpcg_config_parse(json, 4096, &cfg);
    if (rc != WPCG_OK) return rc;
    cfg.max_pos = 2048;
    return wpcg_model_create(ctx, WPCG_SCHEME_V4, &cfg, out);
}
""")
    r = subprocess.run(["gcc", "-std=c11", "-pedantic", "-Wall", "-Wextra", "-Werror", "-I",
                        os.path.dirname(HEADER), "-c", str(src), "-o", str(tmp_path / "cfg.o")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
