"""Resource limits of the built gfx950 kernels, read from the code object's
AMDGPU metadata (no GPU needed).

A GEMM whose accumulators end up in scratch memory still computes the right
result but runs several times slower (the 256x256 QKV GEMM did, once, when its
epilogue loop was left rolled), so the parity tests cannot catch it; this test
does. It also checks the LDS and register budgets the kernels are written for.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "rustane_amd", "libhip_bridge.so")
LLVM = "/opt/rocm/llvm/bin"


def _kernel_metadata():
    bundler = os.path.join(LLVM, "clang-offload-bundler")
    readelf = os.path.join(LLVM, "llvm-readelf")
    objcopy = shutil.which("objcopy") or os.path.join(LLVM, "llvm-objcopy")
    if not (os.path.exists(LIB) and os.path.exists(bundler) and os.path.exists(readelf)):
        pytest.skip("built library or ROCm LLVM tools not present")
    notes = ""
    with tempfile.TemporaryDirectory() as d:
        fat = os.path.join(d, "fat.bin")
        # objcopy rewrites its input file when no output file is named, which
        # would change the library under any process that has it mapped: write
        # the (unused) copy into the temporary directory instead.
        subprocess.run([objcopy, "--dump-section", f".hip_fatbin={fat}", LIB,
                        os.path.join(d, "lib_copy.so")], check=True,
                       capture_output=True)
        # one offload bundle per translation unit, concatenated; the bundler
        # reads only the first bundle of a file, so split them
        data = open(fat, "rb").read()
        magic = b"__CLANG_OFFLOAD_BUNDLE__"
        starts = [i for i in range(len(data)) if data.startswith(magic, i)]
        for n, (a, b) in enumerate(zip(starts, starts[1:] + [len(data)])):
            part, co = os.path.join(d, f"part{n}.bin"), os.path.join(d, f"part{n}.co")
            with open(part, "wb") as f:
                f.write(data[a:b])
            subprocess.run([bundler, "--type=o", "--unbundle", f"--input={part}", f"--output={co}",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950"], check=True,
                           capture_output=True)
            notes += subprocess.run([readelf, "--notes", co], check=True, capture_output=True,
                                    text=True).stdout
    kernels, cur = [], None
    for line in notes.splitlines():
        if line.startswith("  - "):  # a new entry of amdhsa.kernels
            cur = {}
            kernels.append(cur)
            line = "    " + line[4:]
        m = re.match(r"^    \.(\w+):\s+(\S+)", line)
        if cur is not None and m:
            cur[m.group(1)] = m.group(2)
    return [k for k in kernels if "name" in k]


def test_gemm_kernels_keep_accumulators_in_registers():
    ks = _kernel_metadata()
    gemms = [k for k in ks if "gemm_nt_kernel" in k["name"]]
    assert len(gemms) >= 7, "expected the GEMM tile instantiations in the library"
    for k in gemms:
        # a few spilled address registers outside the main loop are tolerated;
        # an accumulator tile in scratch would be >= 1 KiB
        assert int(k["private_segment_fixed_size"]) <= 128, (k["name"], k["private_segment_fixed_size"])


def test_kernels_fit_the_cu():
    for k in _kernel_metadata():
        assert int(k["group_segment_fixed_size"]) <= 160 * 1024, k["name"]
        assert int(k["vgpr_count"]) <= 512, k["name"]
        assert k.get("uses_dynamic_stack", "false") == "false", k["name"]
