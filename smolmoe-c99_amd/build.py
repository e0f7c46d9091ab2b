"""Builds libsmq_gfx950.so (hipcc, gfx950 only) and the C host forward pass
libsmq_model.so (gcc, linked against it) in place.

Flags that the arithmetic contract depends on:
  -ffp-contract=off                        no a*b+c fused into an FMA
  -fhip-fp32-correctly-rounded-divide-sqrt correctly rounded amax/127, 1/scale
  -fno-gpu-flush-denormals-to-zero         f32 denormals kept (tiny scales)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                           no packed f32 math in device code
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libsmq_gfx950.so")
SOURCES = [os.path.join(HERE, "csrc", f) for f in ("smq_kernels.hip", "smq_gemv.hip", "smq_decode.hip", "smq_mfma.hip", "smq_fused.hip", "smq_convert.hip",
                                                     "smq_anchor.hip", "smq_api.cpp")]
HEADERS = [os.path.join(HERE, "csrc", "smq_internal.h"), os.path.join(HERE, "csrc", "smq_device.h"),
           os.path.join(ROOT, "include", "smq.h")]
OBJ_DIR = os.path.join(HERE, "_build")
MODEL_LIB = os.path.join(HERE, "libsmq_model.so")
MODEL_SOURCES = [os.path.join(HERE, "host", "smq_model.c"), os.path.join(HERE, "host", "smq_synth.c")]
# The host side keeps IEEE double/float as written (RoPE tables in double).
MODEL_FLAGS = ["-std=c99", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-Wextra",
               "-Werror"]

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def _quiet(text):
    """hipcc's host pass does not know the packed-fp32 feature: that note is harmless."""
    return "\n".join(line for line in text.splitlines() if "packed-fp32-ops" not in line)


def build(verbose=False):
    """Compiles each source to an object in parallel, then links the library."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc")]
    compile_flags = [f for f in FLAGS if f != "-shared"]
    jobs = []
    for src in SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
        cmd = [hipcc()] + compile_flags + inc + ["-c", src, "-o", obj]
        jobs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = False
    for src, obj, proc in jobs:
        out = _quiet(proc.communicate()[0])
        if proc.returncode != 0:
            sys.stderr.write(out + "\n")
            failed = True
        elif verbose and out.strip():
            sys.stderr.write(out + "\n")
    if failed:
        raise RuntimeError("hipcc failed building libsmq_gfx950.so")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB + ".tmp"] + [obj for _, obj, _ in jobs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(_quiet(res.stdout + res.stderr) + "\n")
        raise RuntimeError("hipcc failed linking libsmq_gfx950.so")
    os.replace(LIB + ".tmp", LIB)
    cmd = [os.environ.get("CC", "gcc")] + MODEL_FLAGS + ["-I", os.path.join(ROOT, "include"), "-o",
                                                         MODEL_LIB + ".tmp"] + MODEL_SOURCES + \
        ["-L", HERE, "-lsmq_gfx950", "-Wl,-rpath,$ORIGIN", "-lm", "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr + "\n")
        raise RuntimeError("gcc failed building libsmq_model.so")
    os.replace(MODEL_LIB + ".tmp", MODEL_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
