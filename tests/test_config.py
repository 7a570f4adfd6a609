"""Plan selection and validation (host logic), following reskv tests/test_config.py.

The golden answers below are the reference's own known-answer tests
(tests/test_config.py:31-42, 91-114) plus the full resolve table of
reskv/config.py:166-217 evaluated by hand.
"""

import subprocess
import sys
from pathlib import Path

import pytest

from reskv_amd import KernelPlan, ResKVKernelConfig
from reskv_amd.config import _model_settings


@pytest.mark.parametrize(
    "settings",
    [
        {"sparsity": 0.25},
        {"bits": 8},
        {"layout": "invalid"},
        {"rope_mode": "invalid"},
        {"sparsity": 0.5, "layout": "structured"},
        {"bits": 2, "layout": "structured", "sparsity": 0.75},
        {"bits": 16, "layout": "tiled", "sparsity": 0.75},
        {"num_clusters": 65},
        {"max_clusters": 0},
        {"group_size": 0},
        {"recent_size": -1},
        {"softmax_mode": "fixed_shift"},
        {"centroid_fusion": "bogus"},
        {"kmeans_iterations": 0},
        {"num_clusters": 1.0},
    ],
)
def test_invalid_config(settings):
    with pytest.raises(ValueError):
        ResKVKernelConfig(**settings)


def test_selection_preserves_distinct_semantics():
    assert ResKVKernelConfig(bits=16, layout="tiled").resolve(1).layout == "tiled"
    assert ResKVKernelConfig(bits=16, layout="auto").resolve(1).layout == "unstructured"
    assert ResKVKernelConfig(bits=16, layout="auto").resolve(16).layout == "unstructured"
    assert ResKVKernelConfig(bits=16, sparsity=0.75, layout="auto").resolve(1).centroid_fusion == "per_token"
    assert ResKVKernelConfig(bits=16, sparsity=0.75, layout="auto").resolve(16).centroid_fusion == "deferred"
    assert ResKVKernelConfig(bits=16, sparsity=0.75).resolve(1).layout == "structured"
    unstructured_int4 = ResKVKernelConfig(bits=4, sparsity=0.75, layout="unstructured")
    assert unstructured_int4.resolve(16).centroid_fusion == "per_token"
    assert ResKVKernelConfig(bits=4, sparsity=0.75, layout="structured").resolve(16).tokens_per_warp == 8


# (sparsity, bits, layout, fusion, batch) -> (layout, fusion, nnz, tpw, splits, fixed)
RESOLVE_TABLE = [
    ((0.5, 16, "auto", "auto", 1), ("unstructured", "deferred", 64, 2, 0, False)),
    ((0.5, 16, "tiled", "auto", 32), ("tiled", "per_token", 64, 4, 0, False)),
    ((0.75, 16, "auto", "auto", 1), ("structured", "per_token", 32, 4, 20, False)),
    ((0.75, 16, "auto", "auto", 2), ("structured", "per_token", 32, 4, 20, False)),
    ((0.75, 16, "auto", "auto", 4), ("structured", "deferred", 32, 4, 20, False)),
    ((0.75, 16, "unstructured", "auto", 8), ("unstructured", "deferred", 32, 2, 0, False)),
    ((0.75, 4, "auto", "auto", 1), ("structured", "per_token", 32, 4, 20, False)),
    ((0.75, 4, "auto", "auto", 4), ("structured", "deferred", 32, 4, 20, False)),
    ((0.75, 4, "auto", "auto", 8), ("structured", "deferred", 32, 8, 14, False)),
    ((0.75, 4, "auto", "auto", 32), ("structured", "deferred", 32, 4, 10, False)),
    ((0.75, 4, "structured", "per_token", 8), ("structured", "per_token", 32, 4, 16, False)),
    ((0.5, 4, "auto", "auto", 2), ("unstructured", "per_token", 64, 16, 40, False)),
    ((0.5, 4, "auto", "auto", 4), ("unstructured", "per_token", 64, 8, 20, False)),
    ((0.5, 4, "auto", "auto", 8), ("unstructured", "per_token", 64, 12, 0, False)),
    ((0.5, 2, "auto", "auto", 16), ("unstructured", "per_token", 64, 16, 0, False)),
    ((0.75, 2, "auto", "auto", 6), ("unstructured", "per_token", 32, 16, 0, False)),
]


@pytest.mark.parametrize("args,expected", RESOLVE_TABLE)
def test_resolve_table(args, expected):
    sparsity, bits, layout, fusion, batch = args
    plan = ResKVKernelConfig(sparsity=sparsity, bits=bits, layout=layout, centroid_fusion=fusion).resolve(batch)
    got = (plan.layout, plan.centroid_fusion, plan.nnz, plan.tokens_per_warp, plan.splits, plan.fixed_shift)
    assert got == expected


def test_fixed_shift_plan():
    cfg = ResKVKernelConfig(sparsity=0.75, bits=4, softmax_mode="fixed_shift")
    assert cfg.resolve(4).fixed_shift is True
    with pytest.raises(ValueError, match="fixed_shift"):
        ResKVKernelConfig(sparsity=0.75, bits=4, softmax_mode="fixed_shift").resolve(1)


@pytest.mark.parametrize(
    "kwargs",
    [
        {"layout": "tiled", "centroid_fusion": "deferred"},
        {"layout": "unstructured", "centroid_fusion": "per_token"},
        {"layout": "unstructured", "bits": 4, "centroid_fusion": "deferred"},
    ],
)
def test_incompatible_fusion_rejected_at_resolve(kwargs):
    with pytest.raises(ValueError):
        ResKVKernelConfig(**kwargs).resolve(1)


def test_config_round_trip():
    cfg = ResKVKernelConfig(bits=16, sparsity=0.75, layout="unstructured", rope_mode="theta")
    assert ResKVKernelConfig(**cfg.to_dict()) == cfg


@pytest.mark.parametrize(
    "changes",
    [
        {"bits": 4.0},
        {"nnz": 64.0},
        {"tokens_per_warp": 2.0},
        {"splits": True},
        {"fixed_shift": 0},
        {"layout": "structured"},
        {"layout": "tiled"},
        {"bits": 4},
        {"fixed_shift": True},
        {"splits": -1},
        {"tokens_per_warp": 3},
    ],
)
def test_invalid_kernel_plan_is_rejected(changes):
    values = ResKVKernelConfig().resolve(1).to_dict()
    with pytest.raises(ValueError):
        KernelPlan(**{**values, **changes})


def test_bit_width_requires_an_integer():
    with pytest.raises(ValueError, match="bits"):
        ResKVKernelConfig(bits=4.0)


@pytest.mark.parametrize("batch_size", [True, 1.5, 0, -3])
def test_batch_size_requires_a_positive_integer(batch_size):
    with pytest.raises(ValueError, match="positive integer"):
        ResKVKernelConfig().resolve(batch_size)


@pytest.mark.parametrize("bits", [2, 4, 16])
@pytest.mark.parametrize("batch_size", [1, 2, 4, 8, 16, 32])
def test_sparse75_default_plan(bits, batch_size):
    settings = ResKVKernelConfig(sparsity=0.75, bits=bits)
    plan = settings.resolve(batch_size)
    assert settings.layout == "auto"
    assert plan.layout == ("unstructured" if bits == 2 else "structured")
    assert plan.centroid_fusion == ("per_token" if bits == 2 or batch_size <= 2 else "deferred")
    assert ResKVKernelConfig(**settings.to_dict()).resolve(batch_size) == plan


@pytest.mark.parametrize("batch_size", [1, 2, 4, 8, 16, 32])
def test_sparse50_default_plan(batch_size):
    settings = ResKVKernelConfig(sparsity=0.5, bits=16)
    plan = settings.resolve(batch_size)
    assert (plan.layout, plan.centroid_fusion) == ("unstructured", "deferred")
    assert ResKVKernelConfig(sparsity=0.5, bits=16, layout="unstructured").resolve(batch_size) == plan
    tiled = ResKVKernelConfig(sparsity=0.5, bits=16, layout="tiled").resolve(batch_size)
    assert (tiled.layout, tiled.centroid_fusion) == ("tiled", "per_token")


@pytest.mark.parametrize(
    "plan_kwargs,width,meta",
    [
        (dict(sparsity=0.5), 64, (2, "int64")),
        (dict(sparsity=0.75, layout="unstructured"), 32, (2, "int64")),
        (dict(sparsity=0.5, layout="tiled"), 64, (4, "int32")),
        (dict(sparsity=0.75), 32, (4, "int32")),
        (dict(sparsity=0.75, bits=4), 4, (2, "int32")),
        (dict(sparsity=0.5, bits=4), 16, None),
        (dict(sparsity=0.5, bits=2), 8, None),
    ],
)
def test_storage_contract(plan_kwargs, width, meta):
    plan = ResKVKernelConfig(**plan_kwargs).resolve(4)
    assert plan.payload_width == width
    assert plan.metadata_spec == meta


def test_model_settings_round_trip():
    from types import SimpleNamespace

    holder = SimpleNamespace()
    cfg = ResKVKernelConfig(sparsity=0.75, bits=4, num_clusters=4, max_clusters=8)
    assert _model_settings(holder, cfg, ResKVKernelConfig, "reskv_kernel_config") == cfg
    assert _model_settings(holder, None, ResKVKernelConfig, "reskv_kernel_config") == cfg
    with pytest.raises(TypeError, match="expected ResKVKernelConfig"):
        _model_settings(holder, object(), ResKVKernelConfig, "reskv_kernel_config")


@pytest.mark.parametrize("stored", [False, 0, "", [], {"unknown": 1}])
def test_invalid_saved_configuration_is_not_replaced_with_defaults(stored):
    from types import SimpleNamespace

    holder = SimpleNamespace(reskv_kernel_config=stored)
    with pytest.raises(ValueError, match="checkpoint compression settings"):
        _model_settings(holder, None, ResKVKernelConfig, "reskv_kernel_config")


def test_import_does_not_initialize_torch_or_the_library():
    subprocess.run(
        [
            sys.executable,
            "-c",
            "import sys; import reskv_amd; assert 'torch' not in sys.modules; "
            "assert reskv_amd.ResKVKernelConfig().bits == 16; "
            "assert 'torch' not in sys.modules",
        ],
        check=True,
        cwd=str(Path(__file__).resolve().parents[1]),
    )


def test_compress_rejects_other_configuration_types():
    from reskv_amd import compress

    for bad in (False, 0, {}, object()):
        with pytest.raises(TypeError, match="compress requires ResKVKernelConfig"):
            compress(None, None, bad)
