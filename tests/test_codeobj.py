"""The built gfx950 code objects (CPU test: reads the library file only).

Every kernel of libortho_amd.so must run without a private segment: a
kernel that needs one has spilled registers or moved a local (typically its
argument struct, after an index computed at run time into it) to scratch
memory, which costs the decode kernel several times its launch time."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "libortho_amd", "libortho_amd.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name):
    p = os.path.join(LLVM, name)
    return p if os.path.exists(p) else shutil.which(name)


def code_object_notes(tmp_path):
    objcopy, bundler, readelf = _tool("llvm-objcopy"), _tool("clang-offload-bundler"), _tool("llvm-readelf")
    if not (objcopy and bundler and readelf):
        pytest.skip("ROCm LLVM tools not found")
    if not os.path.exists(LIB):
        pytest.skip("libortho_amd.so is not built")
    fat = tmp_path / "fat.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", LIB, str(tmp_path / "lib.tmp")], check=True,
                   capture_output=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    notes = []
    for i, o in enumerate(starts):
        b = tmp_path / f"b{i}.bin"
        e = tmp_path / f"b{i}.elf"
        b.write_bytes(data[o:starts[i + 1] if i + 1 < len(starts) else len(data)])
        subprocess.run([bundler, "--unbundle", f"--input={b}", "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={e}"], check=True,
                       capture_output=True)
        notes.append(subprocess.run([readelf, "--notes", str(e)], check=True, capture_output=True,
                                    text=True).stdout)
    return notes


def kernels(notes_text):
    """(name, private segment bytes) of every kernel in one code object's
    metadata note."""
    out = []
    for block in re.split(r"\n\s*- \.", notes_text):
        name = re.search(r"\.name:\s*(\S+)", block)
        priv = re.search(r"\.private_segment_fixed_size:\s*(\d+)", block)
        if name and priv:
            out.append((name.group(1), int(priv.group(1))))
    return out


def test_every_kernel_runs_without_scratch(tmp_path):
    notes = code_object_notes(tmp_path)
    ks = [k for n in notes for k in kernels(n)]
    names = " ".join(n for n, _ in ks)
    for family in ("decode_kernel", "prefill_kernel", "skinny", "mid_kernel", "quarter_kernel", "sieve", "plan"):
        assert family in names, f"no {family} kernels found in the code objects"
    spilled = [(n, p) for n, p in ks if p != 0]
    assert not spilled, f"kernels with a private segment: {spilled[:5]} ({len(spilled)} in all)"
