"""Build librv12.so (the HIP kernels + C ABI) in-tree for gfx950, with a
manifest beside it (librv12.so.build.json: ABI version, sha256 of every
source and header and of the binary, the compiler flags and version) that
ai_amd._lib checks before it loads the library, as the reference binds its
native library only after such a check (ramvi/engine/ramvi_engine/native/
write_manifest.py:1-9, cpu/gcpu.py:121-160).

    python -m ai_amd.build
"""
import hashlib
import json
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "librv12.so")
SOURCES = ["rv12_codec.hip", "rv12_gemv.hip", "rv12_gemm.hip", "rv12_prefill.hip", "rv12_attn.hip", "rv12_static.hip",
           "rv12_api.cpp"]
HEADERS = ["rv12_device.h", "rv12_internal.h"]
MANIFEST = OUT + ".build.json"
PROBE_OUT = os.path.join(HERE, "librv12probe.so")  # bench.py's stream-ceiling probe (not the product)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CODEGEN = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
FLAGS = CODEGEN + ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC]


def _sha256(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def inputs():
    """{relative path: sha256} of every file the library is built from."""
    files = [os.path.join(CSRC, n) for n in SOURCES + HEADERS] + [os.path.join(ROOT, "include", "rv12.h")]
    return {os.path.relpath(f, ROOT): _sha256(f) for f in files}


def abi_version():
    m = re.search(r"#define RV12_ABI_VERSION (\d+)", open(os.path.join(ROOT, "include", "rv12.h")).read())
    return int(m.group(1))


def manifest_problem():
    """None when librv12.so matches its manifest, its sources and the build
    flags of this file; else what does not match."""
    if not os.path.exists(MANIFEST):
        return f"no manifest {MANIFEST}"
    try:
        m = json.load(open(MANIFEST))
    except (OSError, ValueError) as e:
        return f"unreadable manifest {MANIFEST}: {e}"
    if m.get("binary_sha256") != _sha256(OUT):
        return "librv12.so is not the binary its manifest names"
    if m.get("sources") != inputs():
        return "the sources changed since librv12.so was built"
    if m.get("flags") != CODEGEN:
        return "librv12.so was built with other flags"
    if m.get("abi") != abi_version():
        return "include/rv12.h has another ABI version"
    return None


def build(verbose=False):
    tmp = OUT + ".tmp"
    srcs = inputs()  # hashed before the compile reads them
    cmd = [HIPCC] + FLAGS + [os.path.join(CSRC, s) for s in SOURCES] + ["-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "is not a recognized feature")
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if not any(n in l for n in noise))
    if r.returncode:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{msg}")
    if verbose and msg.strip():
        print(msg)
    os.replace(tmp, OUT)
    ver = subprocess.run([HIPCC, "--version"], capture_output=True, text=True).stdout.strip().splitlines()
    man = {"abi": abi_version(), "sources": srcs, "binary_sha256": _sha256(OUT), "flags": CODEGEN,
           "compiler": ver[0] if ver else HIPCC}
    with open(MANIFEST + ".tmp", "w") as f:
        json.dump(man, f, indent=1, sort_keys=True)
    os.replace(MANIFEST + ".tmp", MANIFEST)
    build_probe()
    return OUT


def build_probe():
    """librv12probe.so: the pure-stream probe bench.py times beside the linear."""
    tmp = PROBE_OUT + ".tmp"
    r = subprocess.run([HIPCC] + FLAGS + [os.path.join(CSRC, "rv12_probe.hip"), "-o", tmp], capture_output=True,
                       text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on the probe ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(tmp, PROBE_OUT)


if __name__ == "__main__":
    print(build(verbose=True), file=sys.stderr)
