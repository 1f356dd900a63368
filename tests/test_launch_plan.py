"""The launch plan's bounds (speech.cpp_amd/csrc/spx_plan.h) over a sweep of call sizes, on the CPU: tests/plan_sweep.cpp
built with the host compiler and run. A plan whose chunk index ran past a row's share of the workspace, or whose LDS
regions overlapped, would fault or corrupt another row on the device; this test keeps both off the GPU."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_every_plan_stays_within_the_workspace_and_lds(tmp_path):
    exe = str(tmp_path / "plan_sweep")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include",
                    "-I" + os.path.join(ROOT, "speech.cpp_amd", "csrc"), os.path.join(HERE, "plan_sweep.cpp"), "-o", exe],
                   check=True)
    out = subprocess.run([exe], capture_output=True, text=True)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
