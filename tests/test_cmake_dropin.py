"""The maintainers' HIP CMake stanza, without a GPU: the reference built by
its own CMake with INFERENCE_SDK_BACKEND=HIP registers its 16 GPU-backend
tests; the 11 that do no tensor arithmetic pass through CTest, and
test_tensor_device takes its registered skip code 77. The arithmetic tests run
in test_gpu_cmake_dropin.py."""
import pytest

from tests import cmake_dropin


def test_build_registers_every_gpu_backend_test():
    assert cmake_dropin.registered() == sorted(cmake_dropin.ALL)


@pytest.mark.parametrize("name", cmake_dropin.DEVICE_FREE)
def test_reference_test_passes_through_ctest(name):
    result = cmake_dropin.ctest(name)
    assert result.returncode == 0, (result.stdout, result.stderr)
    assert "100% tests passed" in result.stdout and "Skipped" not in result.stdout


def test_device_test_skips_without_gpu(lib):
    if lib.tensor_device_available():
        pytest.skip("a HIP device is present; test_gpu_cmake_dropin.py runs it")
    result = cmake_dropin.ctest("test_tensor_device")
    assert result.returncode == 0, (result.stdout, result.stderr)
    assert "Skipped" in result.stdout
