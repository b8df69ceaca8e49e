"""bench.py's host-side contract, without a GPU: more than one GPU is refused with a message,
and every mode (the default run and the profiling / sweep modes) reports a missing GPU with
exit status 1 instead of falling back to the CPU."""

import importlib.util
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused(capsys):
    assert _bench().main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU exit")
@pytest.mark.parametrize("argv", [[], ["--decode-sweep"], ["--table-sweep"], ["--profile-kernel", "pool"],
                                  ["--profile-kernel", "dq", "--profile-se"]])
def test_every_mode_needs_a_gpu(capsys, argv):
    assert _bench().main(argv) == 1
    assert "no ROCm GPU visible" in capsys.readouterr().err


def test_unknown_profile_kernel_is_an_argument_error():
    with pytest.raises(SystemExit):
        _bench().main(["--profile-kernel", "nonesuch"])
