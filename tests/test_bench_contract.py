"""bench.py's command-line contract, checked without a GPU: every sub-line
the default run calls exists, and a request for more than one GPU exits
with a message (this build runs on one GPU)."""
from __future__ import annotations

import ast
import json
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent


def test_default_run_calls_only_defined_functions():
    tree = ast.parse((ROOT / "bench.py").read_text())
    defined = {n.name for n in tree.body if isinstance(n, ast.FunctionDef)}
    main = next(n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name == "main")
    called = {n.func.id for n in ast.walk(main)
              if isinstance(n, ast.Call) and isinstance(n.func, ast.Name)}
    for name in ("bench_general", "bench_hybrid", "bench_link", "bench_c4", "bench_thermal",
                 "bench_config", "cpu_baseline", "scalar_floor", "time_steps",
                 "roofline_from_profile", "committed_traffic"):
        assert name in defined, name
    import builtins
    missing = {c for c in called if c not in defined and not hasattr(builtins, c)}
    assert not missing, missing


def test_profile_summaries_parse():
    """The committed kernel summaries the bench lines cite give an average
    duration for their dominant kernel."""
    sys.path.insert(0, str(ROOT))
    import bench
    for summary, kernel in (("engine_kernels_config2_packed.txt", "k_summary"),
                            ("engine_kernels_general.txt", "k_apply"),
                            ("thermal_kernel_grid2048.txt", "k_thermal_march"),
                            ("coupled_kernels_config4.txt", "k_thermal_window")):
        us = bench.profile_kernel_us(summary, kernel)
        assert us is not None and us > 0, (summary, kernel)


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert p.returncode == 2
    line = json.loads(p.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
