"""The C header and the Swift binding over it, checked on the CPU with the
compilers in the image: include/motif_hip.h is plain C99 (and C++), the
CMotifHIP clang module (mlx-motif_amd/swift/CMotifHIP/module.modulemap)
builds and exposes every declared entry point, and each call the Swift
wrapper makes passes as many arguments as the C declaration takes.  No
Swift compiler is in the image, so the wrapper itself is not compiled.
"""

from __future__ import annotations

import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "motif_hip.h"
MODULEMAP = ROOT / "mlx-motif_amd" / "swift" / "CMotifHIP" / "module.modulemap"
SWIFT = ROOT / "mlx-motif_amd" / "swift" / "MotifHIP" / "MotifHIP.swift"
CLANG = shutil.which("clang") or "/opt/rocm/llvm/bin/clang"


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _split_args(s: str) -> list[str]:
    """Top-level comma split of an argument list (nested () and [] kept)."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [a.strip() for a in out]


def _calls(text: str, name_re: str) -> list[tuple[str, list[str]]]:
    """(name, argument list) of every call name_re( ... ) in text."""
    found = []
    for m in re.finditer(name_re + r"\s*\(", text):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        found.append((m.group(1), _split_args(text[m.end():i - 1])))
    return found


def _declarations() -> dict[str, int]:
    """Entry point name -> parameter count, from the header."""
    text = _strip_comments(HEADER.read_text())
    decls = {}
    for name, args in _calls(text, r"\b(motif_[a-z0-9_]+)"):
        decls[name] = 0 if args in ([], ["void"]) else len(args)
    return decls


def _run(cmd, cwd):
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    assert r.returncode == 0, f"{' '.join(map(str, cmd))}\n{r.stdout}\n{r.stderr}"


@pytest.mark.parametrize("std", ["c99", "c11"])
def test_header_is_strict_c(tmp_path, std):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not on PATH")
    _run([gcc, f"-std={std}", "-pedantic-errors", "-Wall", "-Wextra", "-Werror",
          "-fsyntax-only", "-x", "c", str(HEADER)], tmp_path)


def test_header_is_cxx_with_c_linkage(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not on PATH")
    src = tmp_path / "t.cpp"
    names = sorted(_declarations())
    # Every declaration must have C linkage: take each address through an
    # extern "C" function-pointer check.
    src.write_text('#include "motif_hip.h"\n#include <type_traits>\n'
                   + "".join(f"static_assert(std::is_function<decltype({n})>::value, "
                             f'"{n}");\n' for n in names)
                   + "const void* addrs[] = {"
                   + ", ".join(f"(const void*)&{n}" for n in names) + "};\n")
    _run([gxx, "-std=c++11", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
          f"-I{HEADER.parent}", str(src)], tmp_path)
    out = subprocess.run([gxx, "-std=c++11", "-S", "-o", "-", f"-I{HEADER.parent}", str(src)],
                         capture_output=True, text=True, check=True).stdout
    assert "_Z" not in "".join(re.findall(r"\bmotif_\w+|\b_Z\w*motif\w*", out)), \
        "a declaration is missing extern \"C\""


def test_clang_module_builds_and_exports_every_entry_point(tmp_path):
    if not pathlib.Path(CLANG).exists():
        pytest.skip("clang not found")
    names = sorted(_declarations())
    src = tmp_path / "use.m"
    src.write_text("@import CMotifHIP;\n"
                   + "const void* addrs[] = {"
                   + ", ".join(f"(const void*)&{n}" for n in names) + "};\n"
                   + "int main(void) { return motif_abi_version() > 0 ? 0 : 1; }\n")
    _run([CLANG, "-x", "objective-c", "-fmodules", f"-fmodule-map-file={MODULEMAP}",
          f"-fmodules-cache-path={tmp_path / 'cache'}", "-Wall", "-Werror", "-fsyntax-only",
          str(src)], tmp_path)


def test_modulemap_names_the_header_and_library():
    text = MODULEMAP.read_text()
    m = re.search(r'header\s+"([^"]+)"', text)
    assert m and (MODULEMAP.parent / m.group(1)).resolve() == HEADER.resolve()
    assert re.search(r'link\s+"motif_hip"', text)


def test_swift_calls_match_the_c_declarations():
    decls = _declarations()
    text = re.sub(r"//[^\n]*", "", SWIFT.read_text())
    calls = _calls(text, r"\b(motif_[a-z0-9_]+)")
    assert calls, "no C calls found in the Swift wrapper"
    for name, args in calls:
        assert name in decls, f"Swift calls {name}, which the header does not declare"
        assert len(args) == decls[name], (
            f"Swift call of {name} passes {len(args)} arguments, the header takes {decls[name]}")
    # Every decode, attention and RoPE entry point has a Swift face (the RoPE
    # ones through their position-scaled forms, which take scale 1 by default).
    called = {n for n, _ in calls}
    for name in ("motif_sdpa_dual_v", "motif_sdpa_dual_v_q", "motif_gda_decode",
                 "motif_gda_decode_q", "motif_gda_decode_append", "motif_gda_decode_q_append",
                 "motif_gda_decode_heads", "motif_gda_decode_q_heads",
                 "motif_gda_decode_proj_scaled", "motif_gda_decode_q_proj_scaled",
                 "motif_rope_split4_scaled", "motif_gda_prefill_proj_scaled",
                 "motif_gda_post_split", "motif_polynorm", "motif_quant_write4"):
        assert name in called, f"no Swift wrapper calls {name}"


LAYER = SWIFT.parent / "MotifHIPGroupedAttention.swift"


def _swift_funcs(text: str) -> dict[str, list[tuple[str, bool]]]:
    """name -> [(argument label, has default)] of each `static func` of the
    wrapper (labels as a call site writes them)."""
    funcs = {}
    for m in re.finditer(r"static func (\w+)\s*\(", text):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        params = []
        for p in _split_args(text[m.end():i - 1]):
            p = p.strip()
            if not p:
                continue
            head = p.split(":", 1)[0].split()
            params.append((head[0], "=" in p.split(":", 1)[1]))
        funcs[m.group(1)] = params
    return funcs


def test_swift_layer_calls_match_the_wrapper_labels():
    """The layer over the wrapper (MotifHIPGroupedAttention.swift) calls each
    MotifHIP function with its argument labels in declaration order, leaving
    out only defaulted ones -- what the Swift compiler would check."""
    funcs = _swift_funcs(re.sub(r"//[^\n]*", "", SWIFT.read_text()))
    text = re.sub(r"//[^\n]*", "", LAYER.read_text())
    calls = _calls(text, r"\bMotifHIP\.(\w+)")
    assert calls, "no MotifHIP calls found in the layer"
    for name, args in calls:
        assert name in funcs, f"the layer calls MotifHIP.{name}, which the wrapper lacks"
        labels = [a.split(":", 1)[0].strip() for a in args]
        declared = [lab for lab, _ in funcs[name]]
        required = [lab for lab, dflt in funcs[name] if not dflt]
        assert labels == [lab for lab in declared if lab in labels], (
            f"MotifHIP.{name}: labels {labels} out of declaration order {declared}")
        assert set(required) <= set(labels), (
            f"MotifHIP.{name}: missing {sorted(set(required) - set(labels))}")
    called = {n for n, _ in calls}
    for name in ("gdaDecodeFromProjections", "gdaDecodeQuantizedFromProjections",
                 "gdaPrefillFromProjections", "ropeSplit4", "gdaDecode",
                 "gdaDecodeQuantizedAppend", "gdaPostSplit"):
        assert name in called, f"the layer never calls MotifHIP.{name}"
