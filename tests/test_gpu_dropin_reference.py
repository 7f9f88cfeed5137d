"""The drop-in boundary on the GPU: every C test the reference's
CMakeLists.txt registers for a GPU backend, built unmodified against
libinference_sdk_hip.so, passes (test_tensor_device must run, not skip)."""
import pytest

from tests import dropin

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", dropin.ALL)
def test_reference_c_test_passes_on_gpu(name, tmp_path, sdk):
    result = dropin.run(name, str(tmp_path))
    assert result.returncode == 0, (result.stdout, result.stderr)
