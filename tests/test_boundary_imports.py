"""The reference's callers against this package, on the CPU.

* The import statements of pipeline/causal_inference.py:7-10,
  wan/modules/causal_model.py:2-3 and inference.py:191-192 are restated
  here as strings and executed against this package (the reference itself
  is never imported).
* PyramidKVConfig (interface pyramidkv/config.py:56-84): the capacity /
  label known answers of the reference's
  tests/test_pyramidkv_config_robustness.py:15-59, the head-table format
  rules, the out-of-scope head lists (accepted, not loaded) and the
  pipeline's flow (causal_inference.py:707-762: config.capacity_map into
  build_compositions).
* PyramidKVCache / AdaptiveKVCache resolve for imports and isinstance and
  refuse construction with an error naming the MegaCache path.
* The manager's strategy table (pyramidkv_manager.cc:160-214): the known
  answers of tests/test_pyramidkv_manager.py:98-153, on a CPU-resident
  manager.
"""
import csv
import os

import pytest
import torch

CALLER_IMPORTS = {
    "pipeline/causal_inference.py:7-10": (
        "from pyramidkv import AdaptiveKVCache, PyramidKVCache, PyramidKVConfig\n"
        "from pyramidkv import build_compositions\n"
        "from pyramidkv._mega_cache import build_mega_caches\n"
        "from pyramidkv import _mega_state_ref as _mega_ref\n"
        "max_middle_frames = int(_mega_ref.MAX_T_KEYED)\n"),
    "wan/modules/causal_model.py:2-3": (
        "from pyramidkv.cache import PyramidKVCache\n"
        "from pyramidkv._mega_cache import MegaCache\n"),
    "inference.py:191-192": (
        "from pyramidkv import _ops as _pyramidkv_ops\n"
        "loaded = _pyramidkv_ops._ensure_loaded()\n"),
}


@pytest.mark.parametrize("where", sorted(CALLER_IMPORTS))
def test_caller_import_statements(where):
    ns = {}
    exec(compile(CALLER_IMPORTS[where], where, "exec"), ns)
    if "max_middle_frames" in ns:
        assert ns["max_middle_frames"] == 24
        assert callable(ns["build_mega_caches"]) and callable(ns["build_compositions"])
    if "loaded" in ns:
        assert isinstance(ns["loaded"], bool)


def test_package_exports_reference_names():
    import pyramidkv
    want = ["FrameAnchor", "HeadComposition", "MiddleStrategy", "CyclicStrategy", "LagStrategy", "StrideStrategy",
            "MergeStrategy", "RecentStrategy", "HEAD_LABEL_MAP", "build_compositions", "load_head_labels",
            "PyramidKVConfig", "PyramidKVCache", "AdaptiveKVCache"]
    assert sorted(pyramidkv.__all__) == sorted(want)
    for name in want:
        assert getattr(pyramidkv, name) is not None
    assert pyramidkv.HEAD_LABEL_MAP == {-1: "oscillating", 1: "stable", 2: "stable_sparse"}
    for cls in (pyramidkv.CyclicStrategy, pyramidkv.StrideStrategy, pyramidkv.LagStrategy, pyramidkv.MergeStrategy,
                pyramidkv.RecentStrategy):
        assert issubclass(cls, pyramidkv.MiddleStrategy)
    a = pyramidkv.FrameAnchor(k=torch.zeros(1), v=torch.zeros(1), pos=torch.zeros(1, 3), t=5)
    assert a.t == 5


def test_python_caches_are_out_of_scope():
    from pyramidkv import AdaptiveKVCache, PyramidKVCache
    assert issubclass(AdaptiveKVCache, PyramidKVCache)
    for cls in (PyramidKVCache, AdaptiveKVCache):
        with pytest.raises(NotImplementedError, match="build_mega_caches"):
            cls(config=None, batch_size=1, num_heads=12, head_dim=128, layer_idx=0)
    # the caller's isinstance dispatch (causal_model.py:216-228) sees a MegaCache as neither
    from pyramidkv._mega_cache import MegaCache
    assert not issubclass(MegaCache, PyramidKVCache)


def _write(path, rows):
    with open(path, "w", newline="") as f:
        csv.writer(f).writerows(rows)
    return str(path)


def test_config_unknown_labels_fall_back_to_default_capacity(tmp_path):
    from pyramidkv import PyramidKVConfig
    p = _write(tmp_path / "labels.csv", [["-1", "1", "2", "3"], ["1", "1", "-1", "2"]])
    cfg = PyramidKVConfig(config_path=p, num_layers=2, num_heads=4, default_capacity=100,
                          code_map={"-1": 40, "1": 100})
    assert cfg.get_layer_capacities(0) == [40, 100, 100, 100]
    assert cfg.get_layer_capacities(1) == [100, 100, 40, 100]
    assert cfg.get_layer_labels(0) == [-1, 1, 2, 3]


def test_config_explicit_capacity_triples(tmp_path):
    from pyramidkv import PyramidKVConfig
    p = _write(tmp_path / "caps.csv", [["0", "0", "12"], ["0", "1", "34"], ["1", "0", "56"]])
    cfg = PyramidKVConfig(config_path=p, num_layers=2, num_heads=2, default_capacity=99)
    assert cfg.get_layer_capacities(0) == [12, 34]
    assert cfg.get_layer_capacities(1) == [56, 99]


def test_config_defaults_and_reduction_factor(tmp_path):
    from pyramidkv import PyramidKVConfig
    p = _write(tmp_path / "labels.csv", [["-1", "1", "-1", "1"]])
    cfg = PyramidKVConfig(config_path=p, num_layers=1, num_heads=4, default_capacity=300,
                          strategy_reduction_factor=3)
    assert cfg.code_map == {"-1": 100, "1": 300}
    assert cfg.get_layer_capacities(0) == [100, 300, 100, 300]
    missing = PyramidKVConfig(config_path=str(tmp_path / "absent.csv"), num_layers=2, num_heads=3)
    assert missing.capacity_map.dtype == torch.int32 and (missing.capacity_map == 32768).all()
    assert missing.get_layer_drop_mask(1) == [False] * 3 and missing.get_layer_af_groups(0) == [""] * 3


def test_config_head_table_format(tmp_path):
    """Rows of more than three cells are label-matrix rows (blank cells
    dropped); shorter rows are layer, head, capacity entries, applied before
    the matrix resolves every head; entries outside the model or that do not
    parse are ignored; non-integer labels read as 1 in label_map."""
    from pyramidkv import PyramidKVConfig
    p = _write(tmp_path / "mixed.csv", [["layer", "head", "capacity"], ["0", "1", "7"], ["9", "0", "5"],
                                        ["-1", "", "1", "osc", "2"], ["x", "1"], ["2", "-1", "1", "1"]])
    cfg = PyramidKVConfig(config_path=p, num_layers=3, num_heads=4, default_capacity=90,
                          code_map={"-1": 30, "1": 90, "2": 60})
    assert cfg.get_layer_labels(0) == [-1, 1, 1, 2]  # "osc" is not an integer
    assert cfg.get_layer_capacities(0) == [30, 90, 90, 60]  # the matrix overrides the entry (0, 1) -> 7
    assert cfg.get_layer_capacities(1) == [60, 30, 90, 90]
    assert cfg.get_layer_labels(2) == [1, 1, 1, 1] and cfg.get_layer_capacities(2) == [90] * 4  # uncovered layer
    only = _write(tmp_path / "entries.csv", [["1", "1", "5"], ["0", "3", "8"], ["bad", "0", "1"], ["1", "0"]])
    cfg = PyramidKVConfig(config_path=only, num_layers=2, num_heads=2, default_capacity=11)
    assert cfg.capacity_map.tolist() == [[11, 11], [11, 5]] and cfg.label_map.tolist() == [[1, 1], [1, 1]]
    no_one = _write(tmp_path / "no_one.csv", [["2", "-1", "2", "2"]])
    cfg = PyramidKVConfig(config_path=no_one, num_layers=2, num_heads=4, default_capacity=50, code_map={"-1": 5})
    assert cfg.capacity_map.tolist() == [[50, 5, 50, 50], [50, 50, 50, 50]]


def test_config_compositions_compiled_on_first_read(tmp_path, monkeypatch):
    from pyramidkv import PyramidKVConfig, factory
    cfg = PyramidKVConfig(None, num_layers=30, num_heads=12, head_type_csv_path=factory.SHIPPED_LABELS_CSV)
    assert cfg._compositions is None  # nothing compiled until read
    comps = cfg.compositions
    assert len(comps) == 30 and cfg.policies is comps
    assert PyramidKVConfig(None, num_layers=2, num_heads=2).compositions is None
    def refuse(**kw):
        raise ValueError("unreadable head table")
    monkeypatch.setattr(factory, "build_compositions", refuse)
    bad = _write(tmp_path / "bad.csv", [["1", "1"], ["1", "1"]])
    with pytest.warns(UserWarning, match="head compositions.*unreadable"):
        assert PyramidKVConfig(None, num_layers=2, num_heads=2, head_type_csv_path=bad).compositions is None


def test_config_out_of_scope_head_lists_are_not_loaded(tmp_path):
    """The drop-head, soft-ablate and A-F lists are applied only by the
    reference's per-chunk attention path (wan/modules/attention/core.py:
    260-266,323-350), not by the MegaCache path: they are accepted, warn,
    and leave the masks empty."""
    from pyramidkv import PyramidKVConfig
    from pyramidkv import config as C
    drop = _write(tmp_path / "drop.csv", [["layer", "head"], ["0", "1"]])
    af = _write(tmp_path / "af.csv", [["a", "b"], ["c", "d"]])
    C._warned.clear()
    with pytest.warns(UserWarning, match="ignores it") as rec:
        cfg = PyramidKVConfig(config_path=None, num_layers=2, num_heads=2, drop_heads_csv_path=drop,
                              soft_ablate_heads_csv_path=drop, af_policy_enabled=True, af_csv_path=af)
    assert {str(w.message).split(":")[1].split()[0] for w in rec} == {"drop_heads_csv_path",
                                                                      "soft_ablate_heads_csv_path",
                                                                      "af_policy_enabled"}
    assert not cfg.drop_head_mask.any() and not cfg.soft_ablate_head_mask.any()
    assert cfg.af_group_map == [["", ""], ["", ""]] and cfg.get_layer_af_groups(1) == ["", ""]
    assert cfg.drop_heads_csv_path == drop and cfg.af_policy_enabled and cfg.af_csv_path == af


def test_config_to_compositions_pipeline_flow():
    """causal_inference.py:707-762: a label-matrix config, then
    build_compositions over config.capacity_map; the compositions the config
    compiles itself from the head-type CSV are the same records."""
    from pyramidkv import PyramidKVConfig, build_compositions, factory
    csv_path = factory.SHIPPED_LABELS_CSV
    cfg = PyramidKVConfig(csv_path, num_layers=30, num_heads=12, default_capacity=32760,
                          code_map={"-1": 32760, "1": 32760, "2": 32760}, head_type_csv_path=csv_path,
                          frame_seq_length=1560)
    assert cfg.capacity_map.shape == (30, 12) and (cfg.capacity_map == 32760).all()
    labels = factory.load_head_labels(csv_path, 30, 12)
    assert cfg.label_map.tolist() == labels
    comps = build_compositions(num_layers=30, num_heads=12, capacities=cfg.capacity_map, csv_path=csv_path,
                               **factory.PYRAMID_FORCING_POLICY)
    assert len(comps) == 30 and all(len(r) == 12 for r in comps)
    assert [[c.label for c in r] for r in comps] == labels
    assert cfg.compositions is not None and cfg.policies is cfg.compositions
    assert [[c.label for c in r] for r in cfg.compositions] == labels
    cfg.compositions = cfg.policies = comps  # what the pipeline does next


def _cpu_manager():
    from pyramidkv import _ops
    if not _ops.available():
        pytest.skip("torch binding not built")
    # L=2, H=4, D=16, F=8, sink 2 / middle 4 / recent 2, 2 attend chunks (test_pyramidkv_manager.py:28-42)
    return torch.classes.adahead.PyramidKVCacheManager(2, 4, 16, 8, 2, 4, 2, "cpu", "bfloat16", 2)


def test_manager_shapes_and_initial_state():
    mgr = _cpu_manager()
    pack_tokens = 2 * 4 * (8 + int(mgr.max_merge_blocks())) * 8
    assert tuple(mgr.sink_pool().shape) == (2, 4, 2, 8, 16)
    assert tuple(mgr.middle_pool().shape) == (2, 4, 4, 8, 16)
    assert tuple(mgr.recent_pool().shape) == (2, 4, 2, 8, 16)
    assert tuple(mgr.head_t_table().shape) == (2, 4, 8)
    assert tuple(mgr.strategy().shape) == (2, 4, 8) and mgr.strategy().dtype == torch.int8
    assert tuple(mgr.k_flat_out().shape) == (pack_tokens, 1, 16)
    assert tuple(mgr.cu_seqlens_k().shape) == (2 * 4 + 1,)
    assert (mgr.head_t_table() == -1).all() and (mgr.write_idx() == 0).all() and (mgr.valid_count() == 0).all()


def test_manager_set_strategy_writes_one_slot():
    mgr = _cpu_manager()
    mgr.set_strategy(0, 2, 1, torch.tensor([6, 3, 4], dtype=torch.int8))
    s = mgr.strategy()
    assert s[0, 2].tolist() == [1, 6, 3, 4, 0, 0, 0, 0]
    assert int(s[0, 0, 0]) == 0 and int(s[1, 2, 0]) == 0
    mgr.set_strategy(1, 3, -2, torch.tensor([], dtype=torch.int8))
    assert mgr.strategy()[1, 3].tolist() == [-2, 0, 0, 0, 0, 0, 0, 0]


def test_manager_reset_keeps_strategy():
    mgr = _cpu_manager()
    mgr.set_strategy(0, 0, 2, torch.tensor([6], dtype=torch.int8))
    mgr.write_idx().fill_(7)
    mgr.valid_count().fill_(3)
    mgr.head_t_table().fill_(99)
    mgr.cu_seqlens_k().fill_(11)
    mgr.recent_pos_pool().fill_(5)
    mgr.merge_token_count().fill_(4)
    mgr.reset()
    assert (mgr.write_idx() == 0).all() and (mgr.valid_count() == 0).all()
    assert (mgr.head_t_table() == -1).all() and (mgr.cu_seqlens_k() == 0).all()
    assert (mgr.recent_pos_pool() == 0).all() and (mgr.merge_token_count() == 0).all()
    assert mgr.strategy()[0, 0].tolist() == [2, 6, 0, 0, 0, 0, 0, 0]


def test_manager_set_strategy_validates():
    mgr = _cpu_manager()
    p = torch.tensor([1], dtype=torch.int8)
    with pytest.raises(RuntimeError, match="layer_idx out of range"):
        mgr.set_strategy(99, 0, 0, p)
    with pytest.raises(RuntimeError, match="head_idx out of range"):
        mgr.set_strategy(0, 99, 0, p)
    with pytest.raises(RuntimeError, match="must be int8"):
        mgr.set_strategy(0, 0, 0, torch.tensor([1], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="longer than 7"):
        mgr.set_strategy(0, 0, 0, torch.zeros(8, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="int8 range"):
        mgr.set_strategy(0, 0, 300, p)
