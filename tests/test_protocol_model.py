"""CPU model of the decode kernel's tagged dataflow (tests/protocol/dataflow_model.cpp),
built with ThreadSanitizer.

The reference synchronises its phases with grid barriers
(/root/reference/src/barriers.cuh:38-73), whose invariants are no early
release and no lost arrival.  This build replaces them with tagged words; the
model runs the kernel's phase structure, encodings and tag arithmetic (the
kernel's own mk_protocol.h) on 20 threads, 4 of them with no layer role (LM
head only), with randomised delays and checks the equivalent invariants: a
consumer never accepts a stale or aliased word (every value is a known
function of token, layer and index), every wait ends, no data race (TSan), and
a lost word makes every thread unwind through the bounded-wait error path.
Two planted mistakes must be caught: 4-bit tags that repeat every layer, and
role-less workgroups that poll the packed residual stream without first
waiting for the last layer's QKV output.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "protocol", "dataflow_model.cpp")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("dfm") / "dataflow_model")
    subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-fsanitize=thread", "-pthread", SRC, "-o", out],
                   check=True, capture_output=True, text=True, timeout=300)
    return out


def _run(model, *args):
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    return subprocess.run([model, *args], capture_output=True, text=True, timeout=300, env=env)


def test_dataflow_no_stale_values_no_races(model):
    r = _run(model)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-2000:]
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    assert "wrong values 0" in r.stdout and r.stdout.strip().endswith("ok")


def test_lost_word_unwinds_every_thread(model):
    r = _run(model, "drop")
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-2000:]
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    assert "timeout detected" in r.stdout


def test_planted_tag_aliasing_is_caught(model):
    r = _run(model, "alias")
    assert r.returncode == 2, r.stdout + r.stderr[-2000:]
    assert "stale or wrong value" in r.stderr


def test_planted_missing_lm_head_gate_is_caught(model):
    r = _run(model, "nogate")
    assert r.returncode == 2, r.stdout + r.stderr[-2000:]
    assert "x (final)" in r.stderr
