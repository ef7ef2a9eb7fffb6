"""The drop-in boundary: every entry point include/q4kv.h shares with the
reference's src/q4.h has the identical C signature. Both headers are compiled
in one C11 translation unit, where a redeclaration with a different type is a
hard error. Skipped where the reference tree is absent (the GPU box)."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF_H = Path("/root/reference/src/q4.h")
OUR_H = ROOT / "include" / "q4kv.h"


def _decls(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(q4_hip_\w+)\s*\(", text))


@pytest.mark.skipif(not REF_H.exists() or shutil.which("gcc") is None,
                    reason="reference headers or gcc absent")
def test_shared_entry_points_are_type_identical(tmp_path):
    shared = sorted(_decls(REF_H.read_text()) & _decls(OUR_H.read_text()))
    # the decode, append, indexer, prep, GEMV and runtime entries the path uses
    assert len(shared) >= 30, shared
    for name in ("q4_hip_kv_append_d", "q4_hip_qsa_decode_idx", "q4_hip_qsa_decode_n",
                 "q4_hip_f32_to_q8", "q4_hip_qsa_topk_d", "q4_hip_gemv_dd"):
        assert name in shared, name
    src = tmp_path / "both.c"
    lines = [f'#include "{REF_H}"', f'#include "{OUR_H}"']
    # take the address of every shared function through a pointer of the
    # reference's type: a mismatch fails to compile under -Werror
    for n in shared:
        lines.append(f"__typeof__({n}) *const p_{n} = &{n};")
    src.write_text("\n".join(lines) + "\n")
    r = subprocess.run(["gcc", "-std=gnu11", "-fsyntax-only", "-Wall", "-Werror",
                        "-Wno-unused-variable", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
