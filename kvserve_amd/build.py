"""Build libkvhip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m kvserve_amd.build            # compile every source, link kvserve_amd/lib/libkvhip.so

Objects go to kvserve_amd/_build/, the library to kvserve_amd/lib/. Both are git-ignored
build products; the library travels with the source tree so a GPU host needs no compiler.
Each object is compiled with -save-temps, so the gfx950 assembly that the assembler turned into
that very object is kept next to it; it is checked for spill stores the compiler placed where
part of the wave is disabled (kvserve_amd/isa_check.py), and a library with one is not linked.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

if __package__:
    from kvserve_amd import isa_check
else:  # run as a script
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from kvserve_amd import isa_check

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libkvhip.so"
INCLUDE = PKG.parent / "include"

SOURCES = [
    "engine_ops.hip",
    "kvh_api.hip",
    "metadata.hip",
    "paged_attention.hip",
    "paged_attention_f32.hip",
    "probes.hip",
    "reshape_and_cache.hip",
    "rope_and_cache.hip",
]

# Per-source additions. The MFMA kernels treat scores as finite (masked keys become -inf by
# selects, never by arithmetic on NaN), so fmaxf needs no sNaN canonicalisation: without
# -fno-honor-nans every max of an MFMA result costs an extra v_max_f32 x, x, x.
# rope_and_cache reproduces PyTorch's separately rounded multiply and add: no FMA contraction.
SOURCE_FLAGS = {"paged_attention.hip": ["-fno-honor-nans"], "rope_and_cache.hip": ["-ffp-contract=off"]}

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32 (unreliable on these
# hosts); the host pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA sources/results in ordinary VGPRs: the softmax rescale touches the accumulators
    # every chunk, and AGPR copies would cost two moves per accumulator register.
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: libkvhip.so cannot be built")
    return exe


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature; hipcc adds --hip-link to -S runs too
    noise = ("is not a recognized feature for this target", "argument unused during compilation: '--hip-link'")
    err = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if not any(n in line for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_fastcall(verbose: bool = False) -> Path:
    """The CPython binding of the per-step entry points (csrc/pyfast.c -> _kvhfast*.so next to
    this file), compiled with the host compiler; it resolves libkvhip's symbols at run time."""
    import sysconfig

    out = PKG / ("_kvhfast" + sysconfig.get_config_var("EXT_SUFFIX"))
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler for the _kvhfast binding")
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
           str(CSRC / "pyfast.c"), "-ldl", "-o", str(tmp)]  # fmt: skip
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(
    verbose: bool = False, extra_flags: list[str] | None = None, out: Path | None = None, build_dir: Path | None = None
) -> Path:
    """Compile all sources (always; no staleness check) and link the shared library.

    `extra_flags` (e.g. -D tuning macros), `out` and `build_dir` let a tuning sweep build
    variants next to the default kvserve_amd/lib/libkvhip.so."""
    lib = Path(out) if out else LIB
    objdir = Path(build_dir) if build_dir else BUILD
    objdir.mkdir(parents=True, exist_ok=True)
    lib.parent.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    flags = HIP_FLAGS + list(extra_flags or [])

    def compile_one(src: str) -> tuple[Path, Path]:
        # -save-temps=obj keeps the intermediate files next to the object; among them the
        # device assembly that was assembled into this object (no second compilation)
        obj = objdir / (Path(src).stem + ".o")
        asm = objdir / (Path(src).stem + "-hip-amdgcn-amd-amdhsa-gfx950.s")
        asm.unlink(missing_ok=True)
        cmd = [cc, *flags, *SOURCE_FLAGS.get(src, []), f"-I{INCLUDE}", "-save-temps=obj", "-c", str(CSRC / src),
               "-o", str(obj)]  # fmt: skip
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        if not asm.exists():
            raise RuntimeError(f"the device assembly of {src} was not kept ({asm.name})")
        return obj, asm

    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        # the slowest compilation (paged_attention) starts first
        order = sorted(SOURCES, key=lambda s: s != "paged_attention.hip")
        futs = {s: ex.submit(compile_one, s) for s in order}
        built = [futs[s].result() for s in SOURCES]
    objs = [obj for obj, _ in built]
    bad = [f"{asm.name}: {hit}" for _, asm in built for hit in isa_check.check(asm.read_text())]
    if bad:
        raise RuntimeError(
            "the compiler placed spill stores where some lanes are disabled (their reloads would hand those "
            "lanes stale values); change the kernel's register pressure or branch structure:\n" + "\n".join(bad)
        )
    tmp = lib.with_suffix(".so.tmp")
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, lib)  # atomic: a process that already mapped the old file keeps it
    if out is None:
        build_fastcall(verbose)
    return lib


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
