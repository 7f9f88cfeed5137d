#!/usr/bin/env python3
"""Builds the reference with its own CMake and INFERENCE_SDK_BACKEND=HIP.

Test infrastructure: the drop-in check of the boundary, as a maintainer of the
reference would do it.

1. Copies the parts of the reference tree its build reads -- CMakeLists.txt,
   include/, src/, tests/ and the one third-party header a source includes
   (third_party/stb_image.h, from src/common/image.c) -- to a scratch
   directory (the reference itself is read-only and is never built in).
2. Applies the three CMake edits documented for maintainers, read from the
   ```cmake blocks of the integration notes' CMake section (the file named in
   stanza_blocks), so the text tested is the text documented:
   block 1 replaces the backend check's last line, block 2 goes before the
   closing endif() of the backend if-chain (after the METAL branch), block 3
   after the library's compile definitions.
3. Configures (Release, -DINFERENCE_SDK_BACKEND=HIP,
   -DINFERENCE_SDK_HIP_ROOT=<this checkout>) into oracle/_ref/cmake_hip/ and
   builds the library and every registered test, then drops the object files
   (the tests and CTest's files stay; they travel with the tree).

Needs the built HIP library (inference_c_amd/lib/libinference_sdk_hip.so).
Usage: python oracle/cmake_dropin.py [--ref DIR] [--jobs N]
"""
import argparse
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
BUILD = os.path.join(HERE, "_ref", "cmake_hip")
SCRATCH = os.path.join(REPO, "_build", "cmake_ref_src")
CHECK_LAST_LINE = '   NOT INFERENCE_SDK_BACKEND STREQUAL "CUDA")'
METAL_BRANCH = 'elseif(INFERENCE_SDK_BACKEND STREQUAL "METAL")'
DEFINITIONS = ("target_compile_definitions(inference_sdk PUBLIC "
               "INFERENCE_SDK_BACKEND_${INFERENCE_SDK_BACKEND}=1)")


def stanza_blocks():
    """The three ```cmake blocks of the integration notes' CMake section, in order."""
    with open(os.path.join(REPO, "INTEGRATION.md")) as f:
        text = f.read()
    start = text.index("## 2. CMake")
    end = text.index("\n## 3.", start)
    blocks = re.findall(r"```cmake\n(.*?)```", text[start:end], flags=re.S)
    if len(blocks) != 3:
        raise SystemExit(f"INTEGRATION.md section 2 holds {len(blocks)} cmake blocks, not 3")
    return blocks


def patch(cmakelists: str, blocks) -> str:
    lines = cmakelists.split("\n")
    if lines.count(CHECK_LAST_LINE) != 1:
        raise SystemExit("the backend check's last line is not where edit 1 expects it")
    out = []
    metal_seen = branch_done = link_done = False
    for line in lines:
        if line == CHECK_LAST_LINE:
            out.extend(blocks[0].rstrip("\n").split("\n"))
            continue
        if line.strip() == METAL_BRANCH:
            metal_seen = True
        if metal_seen and not branch_done and line == "endif()":
            out.extend(blocks[1].rstrip("\n").split("\n"))
            branch_done = True
        out.append(line)
        if line.strip() == DEFINITIONS:
            out.extend(blocks[2].rstrip("\n").split("\n"))
            link_done = True
    if not (branch_done and link_done):
        raise SystemExit("edit 2 or 3 found no anchor in the reference's CMakeLists.txt")
    return "\n".join(out)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--jobs", type=int, default=min(16, os.cpu_count() or 4))
    args = ap.parse_args()
    if not os.path.isfile(os.path.join(args.ref, "CMakeLists.txt")):
        print(f"reference tree {args.ref} absent: keeping prebuilt {BUILD} (if any)")
        return 0
    hiplib = os.path.join(REPO, "inference_c_amd", "lib", "libinference_sdk_hip.so")
    if not os.path.isfile(hiplib):
        raise SystemExit(f"{hiplib} is missing: build the HIP library first")
    shutil.rmtree(SCRATCH, ignore_errors=True)
    os.makedirs(SCRATCH)
    shutil.copy(os.path.join(args.ref, "CMakeLists.txt"), SCRATCH)
    for sub in ("include", "src", "tests"):
        shutil.copytree(os.path.join(args.ref, sub), os.path.join(SCRATCH, sub), symlinks=True)
    os.makedirs(os.path.join(SCRATCH, "third_party"))
    shutil.copy(os.path.join(args.ref, "third_party", "stb_image.h"),
                os.path.join(SCRATCH, "third_party"))
    path = os.path.join(SCRATCH, "CMakeLists.txt")
    with open(path) as f:
        patched = patch(f.read(), stanza_blocks())
    with open(path, "w") as f:
        f.write(patched)
    shutil.rmtree(BUILD, ignore_errors=True)
    subprocess.run(["cmake", "-S", SCRATCH, "-B", BUILD, "-G", "Unix Makefiles",
                    "-DCMAKE_BUILD_TYPE=Release", "-DINFERENCE_SDK_BACKEND=HIP",
                    f"-DINFERENCE_SDK_HIP_ROOT={REPO}"], check=True)
    subprocess.run(["cmake", "--build", BUILD, "-j", str(args.jobs)], check=True)
    for root, _, files in os.walk(BUILD):
        for name in files:
            if name.endswith(".o"):
                os.remove(os.path.join(root, name))
    return 0


if __name__ == "__main__":
    sys.exit(main())
