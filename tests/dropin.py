"""Runs the reference's own C tests, built unmodified against the HIP library.

`make -C oracle dropin` (run by __graft_entry__.build()) compiles the
reference sources that its CMake build keeps when INFERENCE_SDK_BACKEND=HIP
into an archive and links each test of the reference's CMakeLists.txt:264-317
against that archive and libinference_sdk_hip.so; the binaries sit in
oracle/_ref/dropin/. Each runs in a scratch working directory laid out as the
reference's CTest working directory (a build/ folder for the files the tests
write, tests/fixtures/tokenizer.json), as its CMakeLists.txt:252-257 sets up.
"""
import os
import shutil
import subprocess

from tests.conftest import REPO

DROPIN = os.path.join(REPO, "oracle", "_ref", "dropin")

# Tests that never compute on a TensorBuffer through the library: they pass on
# a machine without a GPU (test_tensor_device returns the reference's skip code
# 77 there).
DEVICE_FREE = ("test_benchmark", "test_json", "test_safetensors", "test_tensor_store",
               "test_tensor_workspace", "test_tensor_prefetch", "test_attention",
               "test_paged_kv_cache", "test_tokenizer", "test_tensor_compute", "test_image")
# Tests that compute on host- or device-storage TensorBuffers; in the HIP build
# that arithmetic runs on the GPU only.
DEVICE = ("test_tensor_buffer", "test_tensor_ops", "test_tensor_graph", "test_tensor_quant",
          "test_tensor_device")
ALL = DEVICE_FREE + DEVICE


def binary(name: str) -> str:
    path = os.path.join(DROPIN, name)
    if not os.path.isfile(path):
        raise FileNotFoundError(f"{path} is missing: build it with `make -C oracle dropin` "
                                "(needs the reference tree and the built HIP library)")
    return path


def run(name: str, workdir, timeout: int = 120) -> subprocess.CompletedProcess:
    exe = binary(name)
    os.makedirs(os.path.join(workdir, "build"), exist_ok=True)
    fixtures = os.path.join(workdir, "tests", "fixtures")
    os.makedirs(fixtures, exist_ok=True)
    shutil.copy(os.path.join(DROPIN, "fixtures", "tokenizer.json"), fixtures)
    print(f"running reference test {name}", flush=True)
    return subprocess.run([exe], cwd=workdir, capture_output=True, text=True, timeout=timeout)
