"""The drop-in boundary without a GPU: the reference's own C tests that do no
tensor arithmetic through the library pass unmodified when linked against
libinference_sdk_hip.so in place of the reference's replaced sources
(workspace-backed tensors, store loads and the prefetcher reach the program's
workspace and store code through the library). The arithmetic tests run in
test_gpu_dropin_reference.py."""
import os

import pytest

from tests import dropin


@pytest.mark.parametrize("name", dropin.DEVICE_FREE)
def test_reference_c_test_passes(name, tmp_path):
    result = dropin.run(name, str(tmp_path))
    assert result.returncode == 0, (result.stdout, result.stderr)


def test_device_test_skips_without_gpu(tmp_path, lib):
    if lib.tensor_device_available():
        pytest.skip("a HIP device is present; test_gpu_dropin_reference.py runs it")
    result = dropin.run("test_tensor_device", str(tmp_path))
    assert result.returncode == 77, (result.stdout, result.stderr)


def test_every_registered_reference_test_is_built():
    built = sorted(n for n in os.listdir(dropin.DROPIN) if n.startswith("test_"))
    assert built == sorted(dropin.ALL)
