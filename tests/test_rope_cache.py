"""RoPE-table cache of the operator layer, on the CPU.

The device table builder is replaced by a CPU stand-in that records each
build, so the tests check the keying and the bounds without a GPU: fresh
inv_freq tensors with equal values share one table, an in-place update of a
caller's tensor is seen, a table grows geometrically and the number of
frequency sets kept is bounded.
"""

import gc

import pytest
import torch

import reskv_amd._extension as ext


@pytest.fixture
def builds(monkeypatch):
    made = []

    def fake_build(freq, count):
        made.append((freq.clone(), count))
        return torch.zeros((count, 128), dtype=torch.float32)

    monkeypatch.setattr(ext, "_build_table", fake_build)
    monkeypatch.setattr(ext, "_ROPE_TABLES", {})
    monkeypatch.setattr(ext, "_BY_TENSOR", {})
    monkeypatch.setattr(ext, "_RETIRED", [])
    return made


def _freq(theta=500000.0, dtype=torch.float32):
    return (theta ** (-torch.arange(64).float() / 64)).to(dtype)


def test_fresh_tensors_with_equal_values_share_one_table(builds):
    base = _freq(dtype=torch.float16)
    tables = set()
    for _ in range(50):
        freq, table = ext._rope(base.float(), 10000.0, "cpu", 2048)  # a new fp32 tensor per call
        tables.add(table.data_ptr())
        assert freq.dtype == torch.float32 and torch.equal(freq, base.float())
    gc.collect()
    assert len(builds) == 1 and len(tables) == 1
    assert len(ext._ROPE_TABLES) == 1
    assert len(ext._BY_TENSOR) <= 1  # entries of collected tensors are dropped


def test_in_place_update_is_seen(builds):
    f = _freq()
    _, t0 = ext._rope(f, 10000.0, "cpu", 1024)
    f.mul_(0.5)
    freq, t1 = ext._rope(f, 10000.0, "cpu", 1024)
    assert len(builds) == 2 and t0.data_ptr() != t1.data_ptr()
    assert torch.equal(freq, f)
    assert len(ext._BY_TENSOR) == 1  # the updated tensor replaced its own entry


def test_growth_is_geometric_and_retires_the_old_table(builds):
    f = _freq()
    _, a = ext._rope(f, 10000.0, "cpu", 100)
    _, b = ext._rope(f, 10000.0, "cpu", 1024)
    assert a is b and a.shape[0] == 1024  # at least 1024 positions
    _, c = ext._rope(f, 10000.0, "cpu", 1025)
    assert c.shape[0] == 2048 and ext._RETIRED == [a]
    _, d = ext._rope(f, 10000.0, "cpu", 5000)
    assert d.shape[0] == 8192 and len(ext._RETIRED) == 2
    assert [n for _, n in builds] == [1024, 2048, 8192]


def test_number_of_frequency_sets_is_bounded(builds):
    keep = []
    for i in range(3 * ext._MAX_FREQ_SETS):
        f = _freq(theta=1000.0 + i)
        keep.append(f)
        ext._rope(f, 10000.0, "cpu", 1024)
    assert len(ext._ROPE_TABLES) == ext._MAX_FREQ_SETS
    # the most recent set is still cached; the oldest was evicted and is rebuilt
    ext._rope(keep[-1], 10000.0, "cpu", 1024)
    assert len(builds) == 3 * ext._MAX_FREQ_SETS
    ext._rope(keep[0], 10000.0, "cpu", 1024)
    assert len(builds) == 3 * ext._MAX_FREQ_SETS + 1


def test_theta_sets_are_keyed_by_theta(builds):
    f1, t1 = ext._rope(None, 500000.0, "cpu", 1024)
    f2, t2 = ext._rope(None, 500000.0, "cpu", 1024)
    f3, _ = ext._rope(None, 10000.0, "cpu", 1024)
    assert t1 is t2 and f1 is f2 and len(builds) == 2
    assert torch.allclose(f1, _freq()) and torch.allclose(f3, _freq(10000.0))


def test_rejects_a_wrong_frequency_count(builds):
    with pytest.raises(RuntimeError, match="inv_freq"):
        ext._rope(torch.ones(32), 10000.0, "cpu", 1024)


def test_inference_tensors_are_keyed_without_a_version(builds):
    """Tensors made under torch.inference_mode have no version counter (the
    model patch runs generate under it); they are keyed by address alone."""
    with torch.inference_mode():
        f = _freq()
        freq, t1 = ext._rope(f, 10000.0, "cpu", 1024)
        _, t2 = ext._rope(f, 10000.0, "cpu", 1024)
        _, t3 = ext._rope(_freq(), 10000.0, "cpu", 1024)  # fresh tensor, equal values
    assert t1 is t2 is t3 and len(builds) == 1 and torch.equal(freq, _freq())
