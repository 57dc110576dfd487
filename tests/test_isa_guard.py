"""The built gfx950 code holds no mixed-precision fma that rounds to fp16
(v_fma_mixlo_f16 / v_fma_mixhi_f16).  The compiler forms one from
fp16(fmaf(a, b, c)), rounding the exact result once, where every scorer
contract rounds to fp32 first and then to fp16; the two differ when the fp32
rounding lands on an fp16 midpoint (tests/test_gpu_rounding.py builds such
sums).  Reads the library built in this tree (no GPU needed)."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "laprune_amd" / "_lib" / "liblaprune_hip.so"
LLVM = Path("/opt/rocm/llvm/bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _tool(name):
    p = LLVM / name
    return str(p) if p.exists() else shutil.which(name)


def test_no_fp16_rounding_mixed_fma(tmp_path):
    if not LIB.exists():
        pytest.skip("library not built")
    objcopy, bundler, objdump = (_tool(n) for n in
                                 ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))
    if not (objcopy and bundler and objdump):
        pytest.skip("LLVM tools not found")
    fat = tmp_path / "fatbin.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", str(LIB)], check=True,
                   capture_output=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)] + [len(data)]
    assert len(starts) > 1, "no offload bundle in the library"
    found, n_fn = {}, 0
    for i in range(len(starts) - 1):
        part, co = tmp_path / f"b{i}.bin", tmp_path / f"b{i}.co"
        part.write_bytes(data[starts[i]:starts[i + 1]])
        subprocess.run([bundler, "--unbundle", "--type=o", f"--targets={TARGET}",
                        f"--input={part}", f"--output={co}"], check=True, capture_output=True)
        asm = subprocess.run([objdump, "-d", str(co)], check=True, capture_output=True,
                             text=True).stdout
        fn = None
        for line in asm.splitlines():
            m = re.match(r"^[0-9a-f]+ <(.*)>:", line)
            if m:
                fn = m.group(1)
                n_fn += 1
            elif re.search(r"\bv_(fma|mad)_mix(lo|hi)_f16\b", line):
                found[fn] = found.get(fn, 0) + 1
    assert n_fn > 50, "disassembly found too few kernels"
    assert not found, f"fp16-rounding mixed fma in: {found}"
