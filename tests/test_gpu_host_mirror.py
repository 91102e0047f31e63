"""The C++ host layer (chimere_amd/host/ggml_gpu.hpp: mirror of the reference's
Rust wrappers chimere-server/src/kernels/ggml_gpu.rs and of the layer
sequences of qwen35_model/moe_ffn.rs) on the GPU: its test program
(tests/cpp/test_host_mirror.cpp, built by `make -C chimere_amd`) holds the
V3 launch sequence bit-exact against the fused layer, which the other GPU
tests hold bit-exact against the oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "chimere_amd", "bin", "test_host_mirror")


@pytest.mark.gpu
def test_host_mirror_program():
    assert os.path.exists(BIN), f"{BIN} is missing: run `make -C chimere_amd`"
    print("host mirror program", flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "host mirror ok" in r.stdout, r.stdout[-3000:] + r.stderr[-2000:]


def test_host_library_loads():
    """libchimere_host.so and the test program are built and link (no GPU call)."""
    import ctypes
    lib = os.path.join(ROOT, "chimere_amd", "libchimere_host.so")
    assert os.path.exists(lib) and os.path.exists(BIN)
    ctypes.CDLL(lib)
    out = subprocess.run(["nm", "-DC", lib], capture_output=True, text=True).stdout
    for name in ("chimere::host::ggml_gpu_gemv_q4_0_q8", "chimere::host::MoeLayer::forward_v3",
                 "chimere::host::MoeLayer::forward_ncmoe", "chimere::host::GgmlGpuBuffers::with_moe"):
        assert name in out, name
