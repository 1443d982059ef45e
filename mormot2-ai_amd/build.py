"""Build libmormot_ai_hip.so: the gfx950 code objects (hipcc --genco), embedded
into the host library by .incbin and loaded at run time with
hipModuleLoadData, plus the C++ host code linked against libamdhip64."""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmormot_ai_hip.so")
# IHIP_TRACE=1: a timing build (IHIP_STAMP phase clocks in the kernels) into
# its own library and build folder, loaded when IHIP_LIB names it
TRACE = os.environ.get("IHIP_TRACE") == "1"
if TRACE:
    BUILD = os.path.join(HERE, "_build_trace")
    LIB = os.path.join(HERE, "libmormot_ai_hip_trace.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
# linear.hip is built once per weight type (IHIP_ONLY_FMT), in parallel
LINEAR_FMTS = ["q8_0", "q4_0", "mxfp4", "q5_0", "q5_1", "q4_k", "q6_k", "f32", "bf16", "f16"]
# gemm.hip (the MFMA prefill GEMM) once per quantized weight type
GEMM_FMTS = ["q8_0", "q4_0", "mxfp4", "q5_0", "q5_1", "q4_k", "q6_k", "f32", "bf16", "f16"]
KERNELS = ([("ops", "ops", []), ("deltanet", "deltanet", [])] +
           [("linear_" + f, "linear", ["-DIHIP_ONLY_FMT_" + f.upper()]) for f in LINEAR_FMTS] +
           [("gemm_" + f, "gemm", ["-DIHIP_ONLY_FMT_" + f.upper()]) for f in GEMM_FMTS])
HOST = ["runtime", "backend", "model", "synth", "gguf"]
# host sources compiled as HIP (a device array registered with the runtime)
HOST_HIP = ["static_scratch"]
HIP_FLAGS = ["--genco", "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", CSRC]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
             "-ffp-contract=off", f"-I{ROCM}/include", "-I", CSRC]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def _kernel(spec):
    name, src, defs = spec
    if TRACE:
        defs = defs + ["-DIHIP_TRACE"]
    src = os.path.join(CSRC, "kernels", src + ".hip")
    out = os.path.join(BUILD, name + ".hsaco")
    _run([HIPCC] + HIP_FLAGS + defs + [src, "-o", out])
    return out


def _host(name):
    src = os.path.join(CSRC, "host", name + ".cpp")
    out = os.path.join(BUILD, name + ".o")
    _run(["g++"] + CXX_FLAGS + ["-c", src, "-o", out])
    return out


def _host_hip(name):
    src = os.path.join(CSRC, "host", name + ".hip")
    out = os.path.join(BUILD, name + ".o")
    _run([HIPCC, "-c", "-fPIC", "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
          "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", CSRC, src, "-o", out])
    return out


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 8)) as ex:
        kfut = {k[0]: ex.submit(_kernel, k) for k in KERNELS}
        hfut = [ex.submit(_host, h) for h in HOST] + [ex.submit(_host_hip, h) for h in HOST_HIP]
        cos = {k: f.result() for k, f in kfut.items()}
        objs = [f.result() for f in hfut]
    embed = os.path.join(BUILD, "embed.S")
    with open(embed, "w") as f:
        f.write('\t.section .rodata\n')
        for k, path in cos.items():
            f.write(f'\t.balign 4096\n\t.global ihip_co_{k}_begin\nihip_co_{k}_begin:\n'
                    f'\t.incbin "{path}"\n\t.global ihip_co_{k}_end\nihip_co_{k}_end:\n'
                    f'\t.byte 0\n')
        # the table the runtime walks: (begin, end) of every code object
        f.write('\t.section .data.rel.ro\n\t.balign 8\n\t.global ihip_co_table\nihip_co_table:\n')
        for k in cos:
            f.write(f'\t.quad ihip_co_{k}_begin, ihip_co_{k}_end\n')
        f.write(f'\t.global ihip_co_count\nihip_co_count:\n\t.long {len(cos)}\n')
        f.write('\t.section .note.GNU-stack,"",@progbits\n')
    tmp = LIB + ".tmp"
    _run(["g++", "-shared", "-o", tmp] + objs + [embed, f"-L{ROCM}/lib", "-lamdhip64",
          f"-Wl,-rpath,{ROCM}/lib", "-lpthread"])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
