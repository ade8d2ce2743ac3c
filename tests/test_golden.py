"""CPU: the oracle reproduces the committed golden fixtures (tests/golden/,
written by tests/golden/make_golden.py), so any later change to the oracle's
math shows up here."""
from pathlib import Path

import numpy as np

import importlib.util

GOLD = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLD / "make_golden.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_small_step_fixture():
    want = np.load(GOLD / "small_step.npz")
    got = _maker().small_step()
    assert abs(float(got["loss"]) - float(want["loss"])) < 1e-5
    g, w = got["grads"].astype(np.float64), want["grads"].astype(np.float64)
    assert np.linalg.norm(g - w) / np.linalg.norm(w) < 1e-5
    p, q = got["params_l0_after"], want["params_l0_after"]
    assert np.linalg.norm(p - q) / np.linalg.norm(q) < 1e-6


def test_tiny_step_fixture():
    want = np.load(GOLD / "tiny_step.npz")
    got = _maker().tiny_step()
    assert abs(float(got["loss"]) - float(want["loss"])) < 1e-12
    assert np.linalg.norm(got["grads"] - want["grads"]) / np.linalg.norm(want["grads"]) < 1e-10


def test_quant_fixture_bit_exact():
    want = np.load(GOLD / "quant.npz")
    from oracle.quant import quantize_rows
    q, s = quantize_rows(want["w"])
    assert np.array_equal(q, want["q"])
    assert np.array_equal(s.view(np.uint32), want["scale"].view(np.uint32))
