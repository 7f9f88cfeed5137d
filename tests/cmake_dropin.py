"""Runs the reference's registered C tests from its own CMake build with
INFERENCE_SDK_BACKEND=HIP (oracle/cmake_dropin.py builds it into
oracle/_ref/cmake_hip/, applying the maintainers' three CMake edits to a
scratch copy of the reference). Each test runs through that build's own
CTest, with the working directory and skip code its CMakeLists.txt:245-317
registers."""
import os
import subprocess

from tests.conftest import REPO
from tests.dropin import ALL, DEVICE, DEVICE_FREE  # noqa: F401  (the same 16 tests)

BUILD = os.path.join(REPO, "oracle", "_ref", "cmake_hip")


def registered() -> list:
    """The test names CTest knows in the build (ctest -N)."""
    out = subprocess.run(["ctest", "--test-dir", BUILD, "-N"], capture_output=True, text=True,
                         timeout=60, check=True).stdout
    return sorted(line.split(":", 1)[1].strip() for line in out.splitlines()
                  if line.strip().startswith("Test") and "#" in line)


def ctest(name: str, timeout: int = 180) -> subprocess.CompletedProcess:
    if not os.path.isfile(os.path.join(BUILD, "CTestTestfile.cmake")):
        raise FileNotFoundError(f"{BUILD} is missing: build it with `python oracle/cmake_dropin.py`"
                                " (needs the reference tree and the built HIP library)")
    print(f"ctest: reference test {name} (CMake build, INFERENCE_SDK_BACKEND=HIP)", flush=True)
    return subprocess.run(["ctest", "--test-dir", BUILD, "-R", f"^{name}$", "--output-on-failure"],
                          capture_output=True, text=True, timeout=timeout)
