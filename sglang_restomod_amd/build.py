"""Build libmi355x_attn.so in-tree from csrc/*.hip with hipcc for gfx950.

    python -m sglang_restomod_amd.build        (or __graft_entry__.build())

Each source compiles to an object under csrc/_build/ in parallel, then one
hipcc link produces sglang_restomod_amd/libmi355x_attn.so. The measurement
kernels of csrc/calibrate/ link into libma_calibrate.so (used by bench.py only). Packed fp32 VALU
instructions are disabled for device code (-packed-fp32-ops).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libmi355x_attn.so"
# measurement kernels for bench.py, linked apart from the attention library
CALIB_SRC = CSRC / "calibrate"
CALIB_OUT = PKG / "libma_calibrate.so"
ARCH = os.environ.get("MI355X_ATTN_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++20",
        "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{PKG.parent / 'include'}",
    ]


# Flags of single sources. The decode/verify kernels (splitkv, paged_any) hold their MFMA
# accumulators in ordinary VGPRs: with them in AGPRs, the online-softmax rescale (VALU,
# which cannot address AGPRs) made the register allocator copy the whole output block
# between the two register files on every key tile (hundreds to thousands of
# v_accvgpr moves per kernel).
_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCE_FLAGS = {"paged_any": _VGPR_FORM, "splitkv": _VGPR_FORM}


def _flags(src: Path, extra: list[str]) -> list[str]:
    return [*common_flags(), *SOURCE_FLAGS.get(src.stem, []), *extra]


def _compile(src: Path, obj: Path, extra: list[str]) -> tuple[Path, str]:
    cmd = [hipcc(), *_flags(src, extra), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj, proc.stderr


def _assembly(src: Path, extra: list[str]) -> Path:
    """Device assembly of `src` (for the static checks)."""
    asm = CSRC / "_build" / (src.stem + ".s")
    cmd = [hipcc(), *_flags(src, extra), "-S", "--cuda-device-only", str(src), "-o", str(asm)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"assembly generation failed: {' '.join(cmd)}\n{proc.stderr}")
    return asm


def verify_assembly(src: Path, asm: Path) -> None:
    """Fail on scalar-cache writes in any kernel, and on in-flight register hazards in
    sources whose kernels issue loads as inline assembly (marked `MA_ASM_PIPELINE`)."""
    from . import isa_check

    bad = isa_check.scalar_cache_writes(str(asm))
    if bad:
        raise RuntimeError(f"{src.name}: scalar-cache writes in the generated code: {sorted(set(bad))}")
    if "MA_ASM_PIPELINE" in src.read_text():
        hazards = isa_check.check_file(str(asm))
        if hazards:
            raise RuntimeError(f"{src.name}: {hazards} in-flight register hazards in the generated code "
                               "(python -m sglang_restomod_amd.isa_check on csrc/_build/*.s lists them)")


def build(verbose: bool = False, extra: list[str] | None = None, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path.

    The device assembly of every source is generated alongside and checked
    (verify_assembly); a finding fails the build.
    """
    extra = list(extra or [])
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no sources under {CSRC}")
    bdir = CSRC / "_build"
    bdir.mkdir(exist_ok=True)
    jobs = jobs or min(2 * len(srcs), max(1, (os.cpu_count() or 2) - 1), 8)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, bdir / (s.stem + ".o"), extra) for s in srcs]
        asms = [ex.submit(_assembly, s, extra) for s in srcs]
        for f in futs:
            obj, err = f.result()
            objs.append(obj)
            if verbose and err.strip():
                print(err, file=sys.stderr)
        for src, f in zip(srcs, asms):
            verify_assembly(src, f.result())
    _link(objs, OUT)
    calib = sorted(CALIB_SRC.glob("*.hip"))
    if calib:
        cobjs = []
        for src in calib:
            cobjs.append(_compile(src, bdir / ("calibrate_" + src.stem + ".o"), extra)[0])
            verify_assembly(src, _assembly(src, extra))
        _link(cobjs, CALIB_OUT)
    return OUT


def _link(objs: list[Path], out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
