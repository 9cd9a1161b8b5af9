"""Builds libwillow_hip.so (gfx950) in-tree from csrc/*.hip with hipcc.

    python willow-v2_amd/build.py            # compile every source, link the library
The library lands next to this file's package: willow-v2_amd/gguf/hip/libwillow_hip.so, where the ctypes shim
loads it from.
"""
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJDIR = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "gguf", "hip", "libwillow_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    # no packed fp32 instructions (v_pk_*_f32) anywhere: some of their forms have given wrong results on MI355X.
    # f16 denormals must stay enabled (the default; no -fdenormal-fp-math=preserve-sign or fast-math): the
    # dequantizing kernels feed quantized values to v_fma_mix_f32 as f16 subnormals
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    objects = []
    procs = []
    for src in sources():
        obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
        objects.append(obj)
        cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = False
    for src, p in procs:
        out = p.communicate()[0].decode(errors="replace")
        # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected
        lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if p.returncode != 0:
            failed = True
            print(f"[build] FAILED {os.path.basename(src)}:\n" + "\n".join(lines), file=sys.stderr)
        elif verbose and lines:
            print(f"[build] {os.path.basename(src)}:\n" + "\n".join(lines), file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed; see the messages above")
    tmp = LIBRARY + f".tmp{os.getpid()}"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp], check=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    t = time.time()
    path = build()
    print(f"built {path} in {time.time() - t:.1f}s")
