"""The CPU decoder restatement (oracle/llama_ref.py) against the reference's
own expected outputs for its tiny llama and qwen2 fixtures: the checks of
TestGenerateMatchesOracle and TestGenerateA8 (reference
cmd/mim-run/main_test.go:178-257), with the same tolerances. The expected
logits come from the reference's float64 oracle; the greedy ids are its
picks."""
import numpy as np
import pytest

import fixture_models as fm
import llama_ref


def run_fixture(name, a8, cache_f16):
    """Prompt, then the oracle's continuation step by step; returns the
    prompt logits and each step's logits (before feeding greedy[i])."""
    cfg, tensors, e = fm.load(name)
    dec = llama_ref.Decoder(llama_ref.Model(cfg, tensors), a8=a8, cache_f16=cache_f16, threads=4)
    P = len(e["prompt_ids"])
    prompt = dec.forward(e["prompt_ids"], np.arange(P))
    steps = [prompt[-1]]
    for i, tok in enumerate(e["greedy"][:-1]):
        steps.append(dec.forward([tok], [P + i])[0])
    return e, prompt, steps


@pytest.mark.parametrize("name", fm.FIXTURES)
def test_generate_matches_oracle(name):
    """Fast paths without 8-bit activations: every logit within 2e-5 of the
    largest, and the same greedy picks (main_test.go:178-217)."""
    e, prompt, steps = run_fixture(name, a8=False, cache_f16=False)
    ok, worst, allowed = fm.near(prompt, fm.f32b64(e["prompt_logits"]), 2e-5)
    assert ok, f"prompt logits: {worst} > {allowed}"
    for i, lg in enumerate(steps):
        ok, worst, allowed = fm.near(lg, fm.f32b64(e["greedy_logits"][i]), 2e-5)
        assert ok, f"step {i}: {worst} > {allowed}"
        assert llama_ref.argmax(lg) == e["greedy"][i], f"step {i}"


@pytest.mark.parametrize("cache_f16", [False, True], ids=["f32cache", "f16cache"])
@pytest.mark.parametrize("name", fm.FIXTURES)
def test_generate_a8(name, cache_f16):
    """8-bit activations: the largest |logit difference| from the float64
    oracle within llama.cpp's own (x1.1 with the cache in f16)
    (main_test.go:219-257)."""
    e, prompt, steps = run_fixture(name, a8=True, cache_f16=cache_f16)
    worst = fm.max_diff(prompt, fm.f32b64(e["prompt_logits"]))
    for i, lg in enumerate(steps):
        worst = max(worst, fm.max_diff(lg, fm.f32b64(e["greedy_logits"][i])))
    bound = e["llama_cpp_max_diff"] * (1.1 if cache_f16 else 1.0)
    assert worst <= bound, f"max |logit difference| {worst} > {bound}"


def test_oracle_mutation_is_caught():
    """A planted mistake in the oracle (rope's sign) fails the fixture check,
    so the check above pins the restatement."""
    cfg, tensors, e = fm.load("llama")
    orig = llama_ref.rope

    def bad_rope(x, cos, sin, rotary, interleaved):
        return orig(x, cos, -sin, rotary, interleaved)

    llama_ref.rope = bad_rope
    try:
        dec = llama_ref.Decoder(llama_ref.Model(cfg, tensors), a8=False, threads=4)
        P = len(e["prompt_ids"])
        lg = dec.forward(e["prompt_ids"], np.arange(P))
    finally:
        llama_ref.rope = orig
    ok, _, _ = fm.near(lg, fm.f32b64(e["prompt_logits"]), 2e-5)
    assert not ok
