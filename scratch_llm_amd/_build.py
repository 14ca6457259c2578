"""Build libsqx_hip.so in-tree from the HIP sources under scratch_llm_amd/csrc.

Every ``*.hip`` file is compiled for gfx950 only, in parallel, then linked into one shared library
next to this file. The library links against the HIP runtime that torch ships (same soname as the
system one, so a process that imported torch maps exactly one HIP runtime), with ``--no-undefined``
so a symbol missing from that runtime fails here rather than at load time on the GPU box.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libsqx_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32 from scalar code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _torch_lib_dir() -> str | None:
    try:
        import torch  # noqa: PLC0415

        d = os.path.join(os.path.dirname(torch.__file__), "lib")
        return d if os.path.exists(os.path.join(d, "libamdhip64.so")) else None
    except Exception:  # pragma: no cover - torch is always present in this image
        return None


def _compile(src: Path, obj: Path, hipcc: str) -> None:
    cmd = [hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link ``libsqx_hip.so``. Always rebuilds."""
    hipcc = _hipcc()
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], hipcc), zip(srcs, objs)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    tl = _torch_lib_dir()
    if tl:
        link += [f"-L{tl}", "-lamdhip64", f"-Wl,-rpath,{tl}"]
    link += ["-Wl,--no-undefined"]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(link)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources (python {sysconfig.get_python_version()})")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
