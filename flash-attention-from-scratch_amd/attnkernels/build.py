"""In-tree build of the attnkernels native code for gfx950.

Two artefacts, both next to this file:
  * ``libattnkernels.so``: the HIP kernels and the C-ABI of
    ``include/attnkernels.h``, compiled by hipcc for gfx950 only (no hipify,
    no CUDA headers);
  * ``attnkernels_ext<EXT_SUFFIX>``: the thin torch extension (pybind module
    ``attnkernels_ext``) compiled by g++ against PyTorch-ROCm's headers and
    linked to the library above through an $ORIGIN rpath.

``python -m attnkernels.build`` (with the package directory on sys.path) or
``__graft_entry__.build()`` runs it.
"""
from __future__ import annotations

import hashlib
import json
import os
import re
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
REPO = PKG.parent.parent
INCLUDE = REPO / "include"
OBJ = PKG / "_build"
LIB = PKG / "libattnkernels.so"
EXT_NAME = "attnkernels_ext"
ARCH = os.environ.get("ATTN_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["prefill.hip", "decode.hip", "cache_write.hip", "stream.hip"]
CPP_SOURCES = ["capi.cpp"]

# Packed FP32 VALU ops stay disabled on this pool; hipcc's host pass warns it
# does not know the feature, which is harmless.
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function"]


def ext_path() -> Path:
    return PKG / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the attnkernels HIP library cannot be built")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(map(str, cmd))}\n"
                           f"{r.stdout}\n{r.stderr}")
    if verbose and (r.stdout or r.stderr):
        print(r.stdout, r.stderr, flush=True)
    return r


# Per-kernel resource usage, from the compiler's kernel-resource-usage remarks
# (VGPRs, AGPRs, spills, LDS, waves per SIMD): read by attnkernels.profiling.
RESOURCE_USAGE = OBJ / "resource_usage.json"
_REMARK = re.compile(r"remark:\s+(Function Name|[A-Za-z ]+?)(?: \[[^\]]*\])?: (\S+) \[-Rpass-analysis")


def parse_resource_usage(text):
    """{mangled kernel name: {field: value}} from -Rpass-analysis=kernel-resource-usage output."""
    out, cur = {}, None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key] = int(val) if val.isdigit() else val
    return out


def build_library(verbose=False, extra_flags=()):
    """Compile the HIP kernels + C-ABI into libattnkernels.so."""
    hipcc = _hipcc()
    OBJ.mkdir(exist_ok=True)
    inc = [f"-I{INCLUDE}", f"-I{CSRC}"]
    jobs = []
    for src in HIP_SOURCES:
        jobs.append([hipcc, *HIPCC_FLAGS, *extra_flags, *inc, "-Rpass-analysis=kernel-resource-usage", "-c",
                     CSRC / src, "-o", OBJ / (src + ".o")])
    for src in CPP_SOURCES:
        jobs.append([hipcc, "-O2", "-std=c++17", "-fPIC", "-Wall", *inc, "-x", "c++",
                     "-D__HIP_PLATFORM_AMD__=1", "-I/opt/rocm/include", "-c",
                     CSRC / src, "-o", OBJ / (src + ".o")])
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        results = list(ex.map(lambda c: _run(c, verbose), jobs))
    usage = {}
    for r in results:
        usage.update(parse_resource_usage(r.stderr))
    RESOURCE_USAGE.write_text(json.dumps(usage, indent=1, sort_keys=True) + "\n")
    objs = [OBJ / (s + ".o") for s in HIP_SOURCES + CPP_SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_extension(verbose=False):
    """Compile the torch glue (ext.cpp) and link it to libattnkernels.so."""
    import torch
    from torch.utils import cpp_extension as ce

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    incs = [f"-I{p}" for p in ce.include_paths(device_type="cuda")]
    incs += [f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = ext_path()
    tmp = out.with_name(out.name + ".tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", CSRC / "ext.cpp", "-o", tmp,
           *incs, "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-deprecated-declarations",
           f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
           "-ltorch_hip", f"-L{PKG}", "-lattnkernels", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    """Build both artefacts; always recompiles."""
    digest = sources_digest()
    build_library(verbose)
    build_extension(verbose)
    STAMP.write_text(digest + "\n")
    return LIB, ext_path()


STAMP = OBJ / "sources.sha256"


def sources_digest() -> str:
    """SHA-256 over the names and contents of every source and header the two
    artefacts are built from (this file included: it holds the flags)."""
    h = hashlib.sha256()
    files = sorted(p for d in (CSRC, INCLUDE) for p in d.iterdir() if p.suffix in (".hip", ".cpp", ".hpp", ".h"))
    for p in files + [Path(__file__).resolve()]:
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()


def is_built() -> bool:
    """Both artefacts exist and were built from the sources as they are now
    (a digest written at build time; file times may not survive a copy of the
    tree).  A stale library would run old kernels under current tests."""
    if not (LIB.exists() and ext_path().exists() and STAMP.exists()):
        return False
    return STAMP.read_text().strip() == sources_digest()


if __name__ == "__main__":
    lib, ext = build(verbose="-v" in sys.argv)
    print("built", lib, ext)
