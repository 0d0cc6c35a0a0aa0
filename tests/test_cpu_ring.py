"""The greedy ring's rules (x0ne-engine_amd/csrc/ring.h, the ones the engine's greedy session and
greedy_timed run) driven on the CPU by a model of the ring, after the reference's
the_greedy_ring_never_overwrites_a_token_not_yet_taken (x0ne-core/oracle/tests/cpu_oracle.rs:
566-614): over ahead 1 .. 15 and 1 .. 70 tokens no word is rewritten before it is taken, no step
is launched past the tokens asked, at most `ahead` steps are in flight. A mistake planted in the
rules (a session one step further ahead than asked, a timed loop that overruns the ring) must fail
the model."""
import os
import subprocess

import pytest

from common import ROOT

CSRC = os.path.join(ROOT, "x0ne-engine_amd", "csrc")
MODEL = os.path.join(ROOT, "tests", "cpp", "ring_model.cpp")


def build_and_run(tmp_path, include_dir):
    exe = tmp_path / "ring_model"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", str(include_dir), MODEL, "-o", str(exe)], check=True,
                   capture_output=True, text=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)


def test_the_greedy_ring_never_overwrites_a_token_not_yet_taken(tmp_path):
    r = build_and_run(tmp_path, CSRC)
    assert r.returncode == 0, r.stderr
    print(r.stdout.strip())


@pytest.mark.parametrize("planted", ["launched - taken_m1 <= ahead", "i + 1 - next >= RING + 1"])
def test_the_model_catches_a_rule_that_runs_too_far_ahead(tmp_path, planted):
    """The model is not vacuous: ring.h with one condition loosened (a copy under tmp_path; the
    product's file is untouched) fails it. The session's rule loosened by one step puts ahead + 1
    steps in flight; greedy_timed's keeps one word spare (RING - 1 outstanding), so its rule
    loosened by two steps rewrites a word not yet collected."""
    text = open(os.path.join(CSRC, "ring.h")).read()
    original = {"launched - taken_m1 <= ahead": "launched - taken_m1 < ahead",
                "i + 1 - next >= RING + 1": "i + 1 - next >= RING - 1"}[planted]
    assert original in text
    d = tmp_path / "planted"
    d.mkdir()
    (d / "ring.h").write_text(text.replace(original, planted))
    r = build_and_run(tmp_path, d)
    assert r.returncode != 0, "a loosened rule passed the ring model"
