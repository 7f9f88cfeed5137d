"""bench.py's contract, without a GPU: the step's byte count, the operand
rotation that keeps each step's chain out of the last-level cache, and the
refusal of more than one GPU."""
import json
import os
import subprocess
import sys

import bench
from tests.conftest import REPO


def test_step_bytes_are_the_configs4_algorithmic_bytes():
    # residual + RMSNorm [4096, 2048] f16: x, r read, h, n written, w once
    assert bench.CFG5["cfg5_residual_rms_norm_f16"][0] == 4 * 4096 * 2048 * 2 + 2048 * 2
    # RoPE in place on q, k [4096, 32, 64] f16: read and written once
    assert bench.CFG5["cfg5_rope_f16"][0] == 2 * 2 * 4096 * 32 * 64 * 2
    # SwiGLU [4096, 8192] f16: gate, up read, out written
    assert bench.CFG5["cfg5_swiglu_f16"][0] == 3 * 4096 * 8192 * 2
    # global sum + max of 2^30 f32: read once
    assert bench.CFG5["cfg5_global_sum_max_f32"][0] == 4 * (1 << 30)
    assert sum(v[0] for v in bench.CFG5.values()) == 4_630_515_712


def test_chain_operand_copies_outrun_the_last_level_cache():
    # the chain's operands and outputs in one copy (x, r, h, n, w, q, k, g, u, o)
    per_copy = (4 * 4096 * 2048 + 2048 + 2 * 4096 * 32 * 64 + 3 * 4096 * 8192) * 2
    others = (bench.CHAIN_SETS - 1) * per_copy
    assert others >= 600_000_000, "two uses of one copy must be >= 600 MB of chain traffic apart"
    assert others > 256 * 2 ** 20


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120, cwd=REPO)
    assert out.returncode == 2
    assert "one GPU" in json.loads(out.stdout.strip().splitlines()[-1])["error"]
