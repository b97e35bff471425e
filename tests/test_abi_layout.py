"""The structs of include/pa_mi355x.h against their ctypes mirrors (and the Rust mirrors in the
repository's integration notes): same field names in the same order, same offsets, same sizes.

The header is compiled with gcc into a small program that prints sizeof/offsetof of every field
the header declares; the field lists come from parsing the header itself, so a field added to
the header but not to a mirror fails here.
"""
from __future__ import annotations

import ctypes as C
import json
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from onnxruntime_ep_mlx_amd import _capi as capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "pa_mi355x.h"

# header struct -> ctypes mirror
MIRRORS = {
    "pa_cache": capi.PaCache,
    "pa_batch": capi.PaBatch,
    "pa_attn": capi.PaAttn,
    "pa_paged_attention_node": capi.PaNode,
    "pa_paged_attention_io": capi.PaIO,
    "pa_gqa_node": capi.PaGqaNode,
    "pa_gqa_io": capi.PaGqaIO,
    "pa_node_info": capi.PaNodeInfo,
    "pa_gqa_node_info": capi.PaGqaNodeInfo,
}

NOTES = "INTEGRATION.md"  # the integration notes at the repository root

# header struct -> Rust mirror name in the integration notes
RUST_MIRRORS = {
    "pa_cache": "PaCache",
    "pa_paged_attention_node": "PaNode",
    "pa_paged_attention_io": "PaIo",
}


def header_structs() -> dict[str, list[str]]:
    """Field names of every `typedef struct X { ... } X;` in the header, in order."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} (\w+);", text, flags=re.S):
        name, body = m.group(1), m.group(2)
        assert name == m.group(3)
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            # "int32_t a, b, c" / "const int32_t* x" / "int64_t input_shape[17][4]"
            head, _, rest = decl.partition(",")
            first = re.sub(r"\[.*$", "", head).split()[-1].lstrip("*")
            names = [first] + [re.sub(r"\[.*$", "", r).strip().lstrip("*")
                               for r in rest.split(",") if rest]
            fields.extend(names)
        out[name] = fields
    return out


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not available")
    structs = header_structs()
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "pa_mi355x.h"',
             "int main(void) {", '  printf("{");']
    first = True
    for s, fields in structs.items():
        sep = "" if first else ","
        first = False
        lines.append(f'  printf("{sep}\\"{s}\\": {{\\"size\\": %zu", sizeof({s}));')
        for f in fields:
            lines.append(f'  printf(", \\"{f}\\": %zu", offsetof({s}, {f}));')
        lines.append('  printf("}");')
    lines += ['  printf("}\\n");', "  return 0;", "}"]
    d = tmp_path_factory.mktemp("abi")
    src, exe = d / "layout.c", d / "layout"
    src.write_text("\n".join(lines))
    subprocess.run([gcc, "-std=c11", "-Wall", f"-I{HEADER.parent}", str(src), "-o", str(exe)],
                   check=True)
    return json.loads(subprocess.run([str(exe)], check=True, capture_output=True,
                                     text=True).stdout)


def test_every_header_struct_has_a_mirror():
    assert set(header_structs()) == set(MIRRORS), sorted(header_structs())


@pytest.mark.parametrize("struct", sorted(MIRRORS))
def test_ctypes_mirror_matches_header(struct, c_layout):
    mirror = MIRRORS[struct]
    names = [f[0] for f in mirror._fields_]
    assert names == header_structs()[struct], struct
    layout = c_layout[struct]
    assert C.sizeof(mirror) == layout["size"], (struct, C.sizeof(mirror), layout["size"])
    for name in names:
        assert getattr(mirror, name).offset == layout[name], (struct, name)


def rust_struct_fields(name: str) -> list[str]:
    text = (ROOT / NOTES).read_text()
    m = re.search(r"pub struct " + name + r" \{(.*?)\n\}", text, flags=re.S)
    assert m, f"Rust mirror {name} not found in {NOTES}"
    body = re.sub(r"//[^\n]*", "", m.group(1))
    return re.findall(r"pub (\w+):", body)


@pytest.mark.parametrize("struct", sorted(RUST_MIRRORS))
def test_rust_mirror_in_integration_doc_matches_header(struct):
    assert rust_struct_fields(RUST_MIRRORS[struct]) == header_structs()[struct]
