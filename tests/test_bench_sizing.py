"""bench.py's engines hold every request the run makes of them, under the
driver's own arguments and the defaults (CPU only: sizes, no engine is built)."""
import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("argv", [["--gpus", "1", "--steps", "20", "--warmup", "5"], [],
                                  ["--steps", "1", "--warmup", "0"], ["--steps", "4096", "--warmup", "4096"]])
def test_every_request_fits_its_engine(argv):
    bench = _bench()
    args = bench.parse(argv)
    for leg, plan in bench.sizing(args).items():
        max_new, room = plan["engine"]
        for prompt, new in plan["requests"]:
            assert prompt + new <= max_new + room, (leg, argv, prompt, new, plan["engine"])


def test_headline_times_the_full_workload():
    """Whatever --steps asks, the timed region is the workload's 2048 new tokens."""
    bench = _bench()
    plan = bench.sizing(bench.parse(["--steps", "20", "--warmup", "5"]))["headline"]
    assert (bench.PROMPT, bench.NEW_TOKENS) in plan["requests"]
    assert bench.NEW_TOKENS == 2048 and bench.PROMPT == 64


def test_prompt_prefill_leg_has_its_own_engine():
    bench = _bench()
    plan = bench.sizing(bench.parse(["--steps", "20", "--warmup", "5"]))
    assert max(p for p, _ in plan["prompt_prefill_bs1"]["requests"]) == 512
    # the headline engine alone would not hold the 512-token prompt
    max_new, room = plan["headline"]["engine"]
    assert plan["prompt_prefill_bs1"]["engine"] != plan["headline"]["engine"] or max_new + room >= 513


def test_leg_turns_an_exception_into_an_error_field(monkeypatch):
    bench = _bench()
    monkeypatch.setattr(bench.torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(bench.torch.cuda, "empty_cache", lambda *a, **k: None)

    def boom():
        raise ValueError("prompt 512 + 1 new exceeds this engine's 84 steps")

    out = bench._leg(boom)
    assert out == {"error": "ValueError: prompt 512 + 1 new exceeds this engine's 84 steps"}
    assert bench._leg(lambda x: x + 1, 1) == 2
