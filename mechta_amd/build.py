"""Builds libmechta_kv.so (the HIP path and its C ABI) in-tree for gfx950 with hipcc, and libmkv_probe.so (bench.py's
plain-read and matrix-rate probes, no part of the ABI).

Every HIP source is compiled with -Xclang -target-feature -Xclang -packed-fp32-ops (no packed-FP32 instructions) and
linked into mechta_amd/lib/libmechta_kv.so. The library has no dependency on torch or on oracle/.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUTDIR = os.path.join(HERE, "lib")
LIB = os.path.join(OUTDIR, "libmechta_kv.so")
SOURCES = ["kv_store.cpp", "kv_root.cpp", "kv_append.hip", "kv_produce.hip", "kv_decode.hip", "kv_prefill.hip",
           "kv_attn32.hip", "flint_store.cpp", "flint_kv.hip"]
# prefill: MFMA accumulators in VGPRs, so the rare lazy rescale of O is plain VALU work instead of AGPR round trips;
# flint_kv: the same for the decodes' score accumulators, which the softmax reads every subtile (no accumulator-register
# reads: f16 full-layer decode 20.4-20.5 against 20.8-20.9 us, sliding layer 10.3-10.4 against 10.6-10.7 us)
# kv_prefill, kv_decode, kv_attn32: no NaN handling in fmaxf (masked scores are -inf, never NaN), so max reductions need no canonicalize
# kv_prefill, kv_decode: the max-ilp machine scheduler (in alternating runs: prefill_f32 0.449 against 0.457-0.459 ms
# per 512-token block, prefill_f16 42.6-42.8% against 42.5-42.6% of the f16 peak on one box; cfg1 10.52-10.55 against
# 10.63-10.68 us per step, the cfg2 decode unchanged)
EXTRA = {"kv_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans", "-mllvm",
                            "-amdgpu-sched-strategy=max-ilp"], "kv_decode.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-sched-strategy=max-ilp"],
         "kv_attn32.hip": ["-fno-honor-nans"], "flint_kv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans"],
         "kv_produce.hip": ["-ffp-contract=off"]}
# measurement aid of bench.py (a plain HBM read of a given size), its own library: not part of the KV-cache ABI
PROBE_SRC, PROBE_LIB = "hbm_probe.hip", os.path.join(OUTDIR, "libmkv_probe.so")
ARCH = os.environ.get("MKV_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -amdgpu-kernarg-preload-count: the first kernel arguments arrive in scalar registers at wave launch instead of by a
# load from the kernarg segment (the code object keeps a prologue that loads them where the firmware does not
# preload); measured on the cfg2 step, in alternating runs: decode 25.90-25.97 against 26.05-26.24 us, merge
# 4.22-4.53 against 4.67-5.29 us, cfg1 10.63-11.04 against 10.84-11.32 us
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16", "-Wall", "-Wno-unused-result",
         "-I", os.path.join(HERE, "..", "include")]


def _extra_flags():
    """MKV_EXTRA_FLAGS: extra hipcc flags for development builds only. They are taken only with MKV_DEV_BUILD=1 set as
    well (a warning is printed), and never when they name the packed-FP32 target feature, which every source keeps
    off."""
    extra = os.environ.get("MKV_EXTRA_FLAGS", "").split()
    if not extra:
        return []
    if os.environ.get("MKV_DEV_BUILD") != "1":
        raise RuntimeError("MKV_EXTRA_FLAGS is set without MKV_DEV_BUILD=1: refusing to build a library with "
                           "unreviewed compiler flags")
    if any("packed-fp32" in x for x in extra):
        raise RuntimeError("MKV_EXTRA_FLAGS may not change the packed-FP32 target feature: " + " ".join(extra))
    print("warning: development build with MKV_EXTRA_FLAGS = " + " ".join(extra), file=sys.stderr, flush=True)
    return extra


def _compile(src, verbose):
    obj = os.path.join(OUTDIR, "obj", os.path.splitext(src)[0] + ".o")
    os.makedirs(os.path.dirname(obj), exist_ok=True)
    lang = ["-x", "hip"]
    cmd = [HIPCC] + FLAGS + EXTRA.get(src, []) + _extra_flags() + lang + ["-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    errs = [l for l in r.stderr.splitlines() if "warning" in l and "packed-fp32-ops" not in l]
    if errs and verbose:
        print("\n".join(errs))
    return obj


def build(verbose=False):
    os.makedirs(OUTDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES + [PROBE_SRC]))
    for lib, o in ((LIB, objs[:-1]), (PROBE_LIB, objs[-1:])):
        tmp = lib + ".tmp"
        cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + o
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp, lib)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
