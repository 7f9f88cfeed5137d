"""The maintainers' HIP CMake stanza on the GPU: all 16 tests the reference's
CMakeLists.txt registers for a GPU backend, built by its own CMake with
INFERENCE_SDK_BACKEND=HIP, pass through CTest (test_tensor_device must run,
not skip)."""
import pytest

from tests import cmake_dropin

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", cmake_dropin.ALL)
def test_reference_test_passes_through_ctest_on_gpu(name, sdk):
    result = cmake_dropin.ctest(name)
    assert result.returncode == 0, (result.stdout, result.stderr)
    assert "100% tests passed" in result.stdout and "Skipped" not in result.stdout
