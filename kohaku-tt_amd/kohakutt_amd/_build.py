"""In-tree build of the native parts, gfx950 only.

* ``libkohakutt_amd.so`` -- the HIP kernels and the C ABI (``include/kohakutt_amd.h``),
  built with ``hipcc --offload-arch=gfx950``; no torch.
* ``_torch_ops.so`` -- the torch op registrations (``csrc/torch_ops.cpp``), a host-only
  C++ library linked against torch and ``libkohakutt_amd.so`` and loaded with
  ``torch.ops.load_library``.

Both land next to this file so they travel with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import re
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent  # kohaku-tt_amd/
REPO = ROOT.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
INCLUDE = REPO / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
ARCH = "gfx950"

CAPI_LIB = PKG / "libkohakutt_amd.so"
OPS_LIB = PKG / "_torch_ops.so"

HIP_SOURCES = [
    "capi.hip",
    "norm.hip",
    "attention.hip",
    *[f"attention_d{d}.hip" for d in (32, 64, 96, 128, 192, 256)],
    "attention_pipe.hip",
    "attention_bwd.hip",
]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    # MFMA accumulators in VGPRs (no AGPR <-> VGPR copies around the softmax).
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(map(str, cmd))}\n{out}")
    return out


# Per-source extra flags.  The attention kernels never produce NaN from finite inputs
# (masked logits are -inf or clamped, NaN mask entries are recognised from their bits), so
# max needs no NaN canonicalisation there.
SOURCE_FLAGS = {f"attention_d{d}.hip": ["-fno-honor-nans"] for d in (32, 64, 96, 128, 192, 256, "_pipe")}
# The unit holding the DMA-staged forward kernels also prints the compiler's per-kernel
# resource usage, which check_dma_spills reads.
RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"
SOURCE_FLAGS["attention_d64.hip"] = SOURCE_FLAGS["attention_d64.hip"] + [RESOURCE_REMARKS]

# attn_fwd_kernel<T, D, NQB, MK, RS, TWIDTH, NW> as the Itanium ABI mangles it.
_FWD_KERNEL = re.compile(
    r"attn_fwd_kernelI(DF16b|DF16_|Dh|f)Li(\d+)ELi(\d+)ELi(\d+)ELb([01])ELi(\d+)ELi(\d+)E"
)
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs Spill|ScratchSize \[bytes/lane\]): (\S+)")


def is_dma_forward(mangled: str) -> bool:
    """Whether a forward kernel instantiation stages K / V by LDS DMA: the condition of
    ``fwd_dma`` in ``csrc/attention_kernels.hpp`` (unmasked, 16-bit, padded head dim 64,
    32-key tiles, 32 rows, or 64 rows without row split)."""
    m = _FWD_KERNEL.search(mangled)
    if m is None:
        return False
    t, d, nqb, mk, rs, tw = m.group(1), *map(int, m.group(2, 3, 4, 5, 6))
    return (t != "f" and d == 64 and mk == 0 and tw == 32
            and (nqb == 2 or (nqb == 4 and rs == 0)))


def check_dma_spills(remarks: str) -> int:
    """Fails when a DMA-staged forward kernel spills VGPRs or uses scratch; returns how many
    such kernels the remarks list.

    Those kernels wait for their tile loads with a fixed ``s_waitcnt vmcnt(4)``, which
    counts only the loads the loop issues itself.  A scratch access between a tile's DMA
    and that wait (a VGPR spill reload) would make the wait release early, a silent race.
    SGPR spills go to VGPR lanes and issue no memory instruction."""
    kernels, name = {}, None
    for key, value in _REMARK.findall(remarks):
        if key == "Function Name":
            name = value
            kernels[name] = {}
        elif name is not None:
            kernels[name][key] = int(value)
    dma = {k: v for k, v in kernels.items() if is_dma_forward(k)}
    bad = [k for k, v in dma.items() if v.get("VGPRs Spill", 0) or v.get("ScratchSize [bytes/lane]", 0)]
    if bad:
        raise RuntimeError(
            "DMA-staged forward kernels spill VGPRs or use scratch, which breaks their fixed "
            "vmcnt waits: " + ", ".join(sorted(bad))
        )
    return len(dma)


def build_capi(jobs: int = 8) -> Path:
    """Compiles the HIP kernels and links ``libkohakutt_amd.so``."""
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD / (src + ".o")
        objs.append(obj)
        cmds.append([str(HIPCC), *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        outs = list(pool.map(_run, cmds))
    for src, out in zip(HIP_SOURCES, outs):
        if RESOURCE_REMARKS in SOURCE_FLAGS.get(src, []) and check_dma_spills(out) == 0:
            raise RuntimeError(f"{src}: no DMA-staged forward kernel in the resource remarks")
    tmp = CAPI_LIB.with_suffix(".so.tmp")
    _run([str(HIPCC), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, CAPI_LIB)
    return CAPI_LIB


def _torch_paths():
    import torch
    import torch.utils.cpp_extension as ext

    incs = ext.include_paths()
    libdir = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return incs, libdir, abi


def build_torch_ops() -> Path:
    """Compiles ``csrc/torch_ops.cpp`` into ``_torch_ops.so``."""
    incs, libdir, abi = _torch_paths()
    BUILD.mkdir(exist_ok=True)
    obj = BUILD / "torch_ops.o"
    cxx = os.environ.get("CXX", "g++")
    _run(
        [
            cxx,
            "-O2",
            "-fPIC",
            "-std=c++17",
            "-Wall",
            "-Wno-unused-parameter",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            "-D__HIP_PLATFORM_AMD__=1",
            "-DUSE_ROCM=1",
            *[f"-I{p}" for p in incs],
            f"-I{ROCM / 'include'}",
            f"-I{INCLUDE}",
            "-c",
            str(CSRC / "torch_ops.cpp"),
            "-o",
            str(obj),
        ]
    )
    tmp = OPS_LIB.with_suffix(".so.tmp")
    _run(
        [
            cxx,
            "-shared",
            "-fPIC",
            str(obj),
            "-o",
            str(tmp),
            f"-L{PKG}",
            "-lkohakutt_amd",
            f"-L{libdir}",
            "-ltorch",
            "-ltorch_cpu",
            "-ltorch_hip",
            "-lc10",
            "-lc10_hip",
            f"-L{ROCM / 'lib'}",
            "-lamdhip64",
            "-Wl,-z,defs",
            "-Wl,-rpath,$ORIGIN",
            f"-Wl,-rpath,{libdir}",
            f"-Wl,-rpath,{ROCM / 'lib'}",
        ]
    )
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


def build_all() -> None:
    build_capi()
    build_torch_ops()


if __name__ == "__main__":
    build_all()
    print(f"built {CAPI_LIB} and {OPS_LIB}", file=sys.stderr)
