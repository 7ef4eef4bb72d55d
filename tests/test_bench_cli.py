"""bench.py's command-line contract and argument checks, on the CPU (every
case here returns or raises before any GPU work)."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=300)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_unknown_only_name_is_rejected():
    r = _run("--only", "gemm,nonsense")
    assert r.returncode != 0
    assert "nonsense" in (r.stderr + r.stdout)


@pytest.mark.parametrize("names,word", [(["no_such_variant"], "unknown variant"),
                                        (["mha_d64_causal_ssa"], "not mha_d64_causal_ssa"),
                                        (["mha_d128", "mha_d128_causal"], "not mha_d128_causal"),
                                        (["mha_bwd_dq_d64"], "not mha_bwd_dq_d64")])
def test_compare_rejects_variants_it_does_not_time(names, word):
    with pytest.raises(ValueError, match=word):
        bench.bench_compare(1, 1, names=names)

