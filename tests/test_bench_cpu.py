"""bench.py's host-side bookkeeping (CPU only): counter-derived figures are reported only for the code object they
were measured on, and the CPU baseline names its host."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_counter_figures_are_keyed_to_their_code_object(bench, monkeypatch):
    monkeypatch.setitem(bench.MEASURED, "forward", {"code": "00aa11bb22cc33dd", "traffic": 123, "valu_insts": 4.5})
    assert bench.measured("forward", "traffic", "00aa11bb22cc33dd", 4_194_304) == (123, None)
    v, why = bench.measured("forward", "traffic", "ffffffffffffffff", 4_194_304)
    assert v is None and "stale" in why and "00aa11bb22cc33dd" in why
    v, why = bench.measured("forward", "valu_insts", "00aa11bb22cc33dd", 1000)
    assert v is None and "N = 4,194,304" in why
    monkeypatch.setitem(bench.MEASURED, "gradient", {"code": None, "traffic": None, "valu_insts": None})
    assert bench.measured("gradient", "traffic", "00aa11bb22cc33dd", 4_194_304) == (None, "not measured")


def test_host_info_names_cpu_and_glibc(bench):
    model, glibc = bench.host_info()
    assert model and isinstance(model, str)
    assert glibc.split(".")[0].isdigit()
