"""Writes rollout_c5_fp32_oracle.json: the fp32 oracle rollout's per-step
RMSE / ACC on bench.py's config-5 setup, recorded by
tests/test_gpu_fullsize.py::test_rollout_config5_bench_setup (needs a GPU).

    python tests/golden/make_rollout_golden.py [OUT_PATH]

OUT_PATH defaults to gpurun_out/rollout_c5_fp32_oracle.json (the GPU box's
output folder); copy it to tests/golden/ afterwards."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

if __name__ == "__main__":
    out = os.path.abspath(sys.argv[1] if len(sys.argv) > 1 else
                          os.path.join(ROOT, "gpurun_out", "rollout_c5_fp32_oracle.json"))
    os.makedirs(os.path.dirname(out), exist_ok=True)
    env = dict(os.environ, NSW_GOLDEN_OUT=out)
    golden = os.path.join(ROOT, "tests", "golden", "rollout_c5_fp32_oracle.json")
    if os.path.exists(golden) and os.path.abspath(golden) != out:
        print(f"note: the test also checks the oracle against the committed {golden}")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-s", "-m", "gpu",
                        "tests/test_gpu_fullsize.py::test_rollout_config5_bench_setup"], cwd=ROOT, env=env)
    sys.exit(r.returncode)
