"""Build libfpv2_hip.so (gfx950) in-tree with hipcc.

Usage: ``python flashprefillv2-mlx_amd/build.py [--jobs N] [--verbose]``.
The library lands next to the ``fpv2`` package (``fpv2/libfpv2_hip.so``)
so it travels with the source tree.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
OUT = HERE / "fpv2" / "libfpv2_hip.so"
SOURCES = ["fpv2_abi.cpp", "fpv2_pool.hip", "fpv2_select.hip", "fpv2_attention.hip",
           "fpv2_decoder.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return found


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-I", str(INCLUDE),
        "-I", str(CSRC),
        # Packed fp32 VALU forms are kept out of the generated code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result",
    ]


def _compile(src: str, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *compile_flags(), "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, flush=True)


# Sources whose device assembly must pass check_isa (asm LDS reads), with
# the kernel symbols to check.
CHECKED = {"fpv2_attention.hip": "sparse_attn_kernel", "fpv2_select.hip": "select_own_kernel"}


def _check_isa(src: str, symbol: str, tmp: Path, verbose: bool) -> None:
    """Compile `src` to gfx950 assembly and run the async-LDS-read check."""
    asm = tmp / (Path(src).stem + ".s")
    cmd = [hipcc(), *compile_flags(), "--cuda-device-only", "-S", str(CSRC / src), "-o", str(asm)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src}:\n{res.stdout}{res.stderr}")
    sys.path.insert(0, str(HERE))
    try:
        import check_isa
    finally:
        sys.path.pop(0)
    text = asm.read_text()
    errors = check_isa.check_text(text, symbol)
    if errors:
        raise RuntimeError(f"{src}: asynchronous LDS read check failed "
                           f"({len(errors)} violations):\n" + "\n".join(errors[:20]))
    if verbose:
        print(f"{src}: async LDS reads ok", flush=True)


def build(jobs: int = 4, verbose: bool = False) -> Path:
    tmp = Path(tempfile.mkdtemp(prefix="fpv2_build_"))
    try:
        objs = [tmp / (Path(s).stem + ".o") for s in SOURCES]
        tasks = [lambda so=so: _compile(so[0], so[1], verbose) for so in zip(SOURCES, objs)]
        tasks += [lambda src=src, sym=sym: _check_isa(src, sym, tmp, verbose) for src, sym in CHECKED.items()]
        with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
            list(pool.map(lambda f: f(), tasks))
        tmp_out = OUT.with_suffix(".so.tmp")
        # --no-undefined: a kernel whose host stub was not emitted must fail
        # here, not at load time.
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined",
               *map(str, objs), "-o", str(tmp_out)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
        os.replace(tmp_out, OUT)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return OUT


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    out = build(args.jobs, args.verbose)
    print(f"built {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
