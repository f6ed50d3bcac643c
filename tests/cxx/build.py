"""Builds tests/cxx/libengine_calls.so: engine_calls.cpp (one namespace jllm
call per ec_* function) plus model_registry_stub.cpp (the engine's mapped-
weight registry), linked against genie-ai-runtime_amd/libjllm_hip.so only.
Test infrastructure for the GPU tests of the C++ boundary; run by
__graft_entry__.build() after the library itself."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
LIBDIR = os.path.join(ROOT, "genie-ai-runtime_amd")
OUT = os.path.join(HERE, "libengine_calls.so")


def build():
    tmp = OUT + ".tmp"
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O2", "-fPIC", "-shared", "-I" + os.path.join(ROOT, "include"),
           os.path.join(HERE, "engine_calls.cpp"), os.path.join(HERE, "model_registry_stub.cpp"),
           "-L" + LIBDIR, "-ljllm_hip", "-Wl,-rpath,$ORIGIN/../../genie-ai-runtime_amd", "-Wl,--no-undefined",
           "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("engine_calls build failed:\n" + r.stderr[-4000:])
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
