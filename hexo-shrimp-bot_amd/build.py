"""In-tree build of the native libraries (run by ``__graft_entry__.build()``).

* ``libhexo_encoder.so`` — host C++ (g++), no GPU dependency;
* ``libmantis_hip.so`` — HIP for gfx950 (hipcc --offload-arch=gfx950);
* ``oracle/liboracle.so`` — the CPU oracle used by the tests (gcc).

Every HIP object is compiled with packed-FP32 instruction selection disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
HIP_SOURCES = ["gather_ops.hip", "stone_attention.hip", "hex_message.hip", "fused_linear.hip", "heads.hip",
               "attention_substage.hip", "cell_heads.hip", "latent_mix.hip", "improve.hip", "relay.hip", "attn_backward.hip", "plan.hip", "latent_broadcast.hip",
               "latent_read.hip", "radius_stage.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs (the unified register file), not AGPRs: saves the
    # accvgpr copies between the matrix products and the softmax/epilogue math
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")


def build_encoder() -> Path:
    out = PKG / "libhexo_encoder.so"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall",
          "-o", str(out), str(CSRC / "encoder" / "hexo_encoder.cpp")])
    return out


def build_hip() -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []

    def one(src: str) -> Path:
        obj = BUILD / (Path(src).stem + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / "kernels" / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as pool:
        objs = list(pool.map(one, HIP_SOURCES))
    out = PKG / "libmantis_hip.so"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(out), *map(str, objs)])
    return out


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "liboracle.so"


def build_all() -> list[Path]:
    return [build_encoder(), build_hip(), build_oracle()]


if __name__ == "__main__":
    for p in build_all():
        print(p)
