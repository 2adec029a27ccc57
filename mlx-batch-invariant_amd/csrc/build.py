"""Build the gfx950 kernel library ``libbi_kernels.so`` in-tree (and the small
CPython binding ``_bi_pycall`` of its hottest entry points).

    python mlx-batch-invariant_amd/csrc/build.py [--jobs N] [--verbose]

Every ``*.hip`` file in this directory is compiled with hipcc for gfx950 and
linked into ``mlx_batch_invariant_amd/libbi_kernels.so`` next to the Python
package. The library links the HIP runtime by its SONAME (libamdhip64.so.7),
so inside a process that has imported torch it binds to the runtime torch
already loaded and shares torch's streams and allocations.

Numerics flags are part of the batch-invariance contract and must not be
changed per file: no fp contraction (every fma is explicit), no fast math,
IEEE division and sqrt, denormals kept, and no packed-fp32 instructions.
Per-file flags (EXTRA_FLAGS) only steer register allocation and instruction
scheduling.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent / "mlx_batch_invariant_amd"
OUT = PKG / "libbi_kernels.so"
OBJ = HERE / "_build"

ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]

# Register-allocation flags per source (no effect on numerics). The attention
# kernels keep every MFMA operand and result in ordinary VGPRs rather than the
# accumulation registers: the prefill kernel then needs no register-to-register
# copies between the two files (272 v_accvgpr_read/write in its assembly
# before) and measured 2-4% faster (config-4 B = 1 / 4 / 16, same box: 0.129 /
# 0.381 / 1.416 -> 0.125 / 0.366 / 1.383 ms), decode 0.4-2%. The dense mid-M
# tile measured 3-8% slower with it, so the flag stays per file; the fp32
# attention kernels keep the default (with it one more of them spills).
#
# The 4-bit quantized sources use the memory-clause scheduler (device pass
# only). Its visible change in the decode GEMV is the prologue: every
# kernel-argument load issued before the first wait, where the default waited
# once in between (one more scalar-load round before the first weight
# request). Same-box A/B, 4-bit g64 [14336, 4096], five alternating runs:
# M = 1 / 2 / 4 / 8 medians 10.41 / 11.17 / 11.53 / 13.29 -> 9.89 / 10.72 /
# 11.03 / 12.84 us, M = 16-64 and large M (128 / 512 / 4096) equal. The 8-bit
# kernels (bi_qmm8_*) measured slower with it (8-bit g128, M = 1 / 2: 14.35 /
# 14.59 -> 14.69 / 15.15 us), the dense source too at M = 1 and 4 (4.81 ->
# 5.16 us), and the attention sources equal or slower.
_CLAUSE = ["-Xarch_device", "-mllvm=-misched=gcn-max-memory-clause"]
EXTRA_FLAGS = {
    "bi_attn_bf16": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "bi_attn_f16": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "bi_qmm_bf16": _CLAUSE,
    "bi_qmm_f16": _CLAUSE,
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the kernel library)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; harmless.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def _stale(src: Path, obj: Path) -> bool:
    """An object is stale if it is missing or older than its source, any
    header of this directory or the C ABI header, or this build script."""
    if not obj.exists():
        return True
    deps = [src, Path(__file__), *HERE.glob("*.h"), *(HERE.parent.parent / "include").glob("*.h")]
    return obj.stat().st_mtime < max(d.stat().st_mtime for d in deps)


def build(jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> Path:
    """Compile every source (``incremental``: only stale objects) and link."""
    cc = hipcc()
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(HERE.glob("*.hip"))
    objs = [OBJ / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(8, os.cpu_count() or 1)
    todo = [(s, o) for s, o in zip(srcs, objs) if not incremental or _stale(s, o)]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [cc, *CFLAGS, *EXTRA_FLAGS.get(s.stem, []), "-c", str(s), "-o", str(o)], verbose)
                for s, o in todo]
        for f in futs:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    # -z defs: a kernel whose host stub was not emitted fails here, not at dlopen
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, OUT)
    build_pycall(verbose)
    return OUT


def build_pycall(verbose: bool = False) -> Path:
    """The CPython binding of the hottest entry points (bi_pycall.c), a host-only
    C extension next to the package; it calls the library through addresses
    the package binds at load time, so it needs neither hipcc nor a link to
    libbi_kernels.so."""
    import sysconfig
    out = PKG / ("_bi_pycall" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no C compiler for bi_pycall.c")
    _run([cc, "-O2", "-shared", "-fPIC", "-Wall", "-I", sysconfig.get_paths()["include"], str(HERE / "bi_pycall.c"),
          "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--jobs", type=int, default=None)
    p.add_argument("--verbose", action="store_true")
    p.add_argument("--incremental", action="store_true", help="recompile only objects older than their inputs")
    a = p.parse_args(argv)
    out = build(a.jobs, a.verbose, a.incremental)
    print(f"built {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
