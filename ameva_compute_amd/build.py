"""Builds libameva_hip.so in-tree for gfx950 with hipcc (no CMake, no JIT cache: the .so travels with the tree).

Flags that carry meaning:
  -ffp-contract=off and -fhip-fp32-correctly-rounded-divide-sqrt: the quantizers must round x * id, 1/d and
      127/amax exactly as the CPU does (bit-exact Q8_0 / Q4_0 bytes);
  -Xclang -target-feature -Xclang -packed-fp32-ops: keep hipcc from emitting packed-FP32 VALU ops;
  -mllvm -amdgpu-mfma-vgpr-form: matrix-core results in VGPRs (the epilogues read them with VALU ops; in AGPRs every
      value costs a v_accvgpr_read first: 64 more VALU ops per 32x32 block of four tiles);
  -mllvm -disable-promote-alloca-to-lds: keep per-thread staging structs in registers, not in LDS slices.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libameva_hip.so")
SOURCES = ["amv_runtime.hip", "amv_quant.hip", "amv_mmv.hip", "amv_i2s.hip", "amv_norm.hip", "amv_attn.hip", "amv_fa_prefill.hip", "amv_mmq.hip", "amv_mmq16.hip", "amv_qgemm.hip", "amv_elem.hip", "amv_bitnet.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-disable-promote-alloca-to-lds",
    "-Wall", "-Wno-unused-function",
]


def sources() -> list[str]:
    return [os.path.join(CSRC, s) for s in SOURCES]


def _jobs() -> int:
    return max(1, min(8, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))


def build(verbose: bool = False) -> str:
    from concurrent.futures import ThreadPoolExecutor

    def compile_one(src):
        obj = os.path.join(CSRC, os.path.basename(src) + ".o")
        r = subprocess.run([HIPCC, *FLAGS, "-c", src, "-o", obj], capture_output=True, text=True)
        return src, obj, r

    objs = []
    with ThreadPoolExecutor(_jobs()) as ex:
        for src, obj, r in ex.map(compile_one, sources()):
            if r.returncode != 0:
                sys.stderr.write(r.stdout + r.stderr)
                raise RuntimeError(f"hipcc failed on {src}")
            if verbose:
                sys.stderr.write(r.stderr)
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    # the libraries over libameva_hip.so and the test code object are independent of each other
    with ThreadPoolExecutor(_jobs()) as ex:
        for f in [ex.submit(fn) for fn in (build_plugin, build_amuda, build_runtime, build_bitnet, build_test_kernels)]:
            f.result()
    return LIB


PLUGIN = os.path.join(HERE, "libggml-ameva.so")


def build_plugin() -> str:
    """libggml-ameva.so: the ggml backend plugin over libameva_hip.so. ggml_backend_buffer_init stays undefined and
    binds to the host's libggml-base at load time."""
    src = os.path.join(CSRC, "ggml_ameva.cpp")
    tmp = PLUGIN + ".tmp"
    commit = "unknown"
    try:
        commit = subprocess.run(["git", "-C", HERE, "rev-parse", "--short", "HEAD"], capture_output=True,
                                text=True).stdout.strip() or "unknown"
    except OSError:
        pass
    cmd = [HIPCC, *FLAGS, "-shared", f'-DAMEVA_BUILD_COMMIT="{commit}"', "-o", tmp, src, "-L" + HERE,
           "-lameva_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on ggml_ameva.cpp")
    os.replace(tmp, PLUGIN)
    return PLUGIN


AMUDA = os.path.join(HERE, "libamuda_hip.so")


def build_amuda() -> str:
    """libamuda_hip.so: the amuda / BitNet C ABI subset (include/amuda_hip.h) over libameva_hip.so (host code only)."""
    src = os.path.join(CSRC, "amuda_hip.cpp")
    tmp = AMUDA + ".tmp"
    cmd = [HIPCC, *FLAGS, "-shared", "-o", tmp, src, "-L" + HERE, "-lameva_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on amuda_hip.cpp")
    os.replace(tmp, AMUDA)
    return AMUDA


RUNTIME = os.path.join(HERE, "libac_runtime_hip.so")


def build_runtime() -> str:
    """libac_runtime_hip.so: the ac_runtime C ABI (include/ac_runtime_hip.h) on HIP (host code only)."""
    src = os.path.join(CSRC, "ac_runtime_hip.cpp")
    tmp = RUNTIME + ".tmp"
    cmd = [HIPCC, *FLAGS, "-shared", "-o", tmp, src]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on ac_runtime_hip.cpp")
    os.replace(tmp, RUNTIME)
    return RUNTIME


BITNET = os.path.join(HERE, "libac_bitnet_hip.so")


def build_bitnet() -> str:
    """libac_bitnet_hip.so: the BitNet per-token engine (include/ac_bitnet_engine_hip.h) over libameva_hip.so."""
    src = os.path.join(CSRC, "ac_bitnet_engine.cpp")
    tmp = BITNET + ".tmp"
    cmd = [HIPCC, *FLAGS, "-shared", "-o", tmp, src, "-L" + HERE, "-lameva_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on ac_bitnet_engine.cpp")
    os.replace(tmp, BITNET)
    return BITNET


TEST_KERNELS = os.path.join(os.path.dirname(HERE), "tests", "ac_kernels", "ac_test_kernels.hip")


def build_test_kernels() -> str:
    """The gfx950 code object the ac_runtime tests load (tests/ac_kernels/ac_test_kernels.hsaco)."""
    out = TEST_KERNELS[:-4] + ".hsaco"
    if not os.path.exists(TEST_KERNELS):  # a package installed without its tests
        return ""
    cmd = [HIPCC, "--genco", "--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-o", out + ".tmp", TEST_KERNELS]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc --genco failed on ac_test_kernels.hip")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
