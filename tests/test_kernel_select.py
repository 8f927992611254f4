"""Selection policy of amd_tuned_torch.kernel_select with the timing stubbed (CPU).

Behaviours pinned here are the reference selector's (its tests/test_kernel_select.py):
fastest (not first) wins, decisions cached per key, stride/kind part of the key, declining
candidates lose, a cached winner that declines is evicted and re-contested, all-decline
returns None, the kill switch, reset(), pick_key, numerical verification against the last
(reference) candidate with the RMS-scaled bar, blacklisting, the disk cache format and
its verify-bar versioning, and OOM handling."""
from __future__ import annotations

import json
import warnings

import pytest
import torch

from amd_tuned_torch import kernel_select as ks


@pytest.fixture(autouse=True)
def _clean(monkeypatch, tmp_path):
    monkeypatch.setattr(ks, "_ENABLED", True)
    monkeypatch.setattr(ks, "_VERIFY_ENABLED", False)
    monkeypatch.setattr(ks, "_DISK_CACHE_ENABLED", False)
    monkeypatch.setattr(ks, "_CACHE_DIR", str(tmp_path))
    ks.reset()
    yield
    ks.reset()


@pytest.fixture
def timings(monkeypatch):
    calls: dict = {}

    def install(table):
        def fake_time(fn):
            calls[fn._name] = calls.get(fn._name, 0) + 1
            if fn() is None:
                return None
            return table.get(fn._name)
        monkeypatch.setattr(ks, "_time", fake_time)
        return calls
    return install


def cands(names, declines=(), outputs=None):
    out = []
    for n in names:
        def thunk(n=n):
            if n in declines:
                return None
            return outputs[n] if outputs else f"out:{n}"
        thunk._name = n
        out.append((n, thunk))
    return out


def args(h=8):
    return torch.zeros(1, 4, h, h), torch.zeros(4, 4, 3, 3), 1, 1, 1


def test_fastest_not_first(timings):
    calls = timings({"native.a": 5.0, "native.b": 9.0, "stock": 1.0})
    x, w, s, p, d = args()
    assert ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "native.b", "stock"])) == "out:stock"
    assert calls == {"native.a": 1, "native.b": 1, "stock": 1}


def test_decision_cached_per_shape(timings):
    calls = timings({"native.a": 1.0, "stock": 4.0})
    x, w, s, p, d = args()
    for _ in range(4):
        assert ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"])) == "out:native.a"
    assert calls == {"native.a": 1, "stock": 1}
    assert list(ks.debug_winners().values()) == ["native.a"]
    assert ks.cached("conv2d", x, w, s, p, d) == "native.a"


def test_shape_stride_kind_are_distinct_keys(timings):
    calls = timings({"native.a": 1.0, "stock": 4.0})
    x, w, s, p, d = args()
    ks.pick("conv2d", x, w, 1, p, d, cands(["native.a", "stock"]))
    ks.pick("conv2d", x, w, 2, p, d, cands(["native.a", "stock"]))
    ks.pick("conv3d", x, w, 1, p, d, cands(["native.a", "stock"]))
    ks.pick("conv2d", torch.zeros(1, 4, 16, 16), w, 1, p, d, cands(["native.a", "stock"]))
    assert len(ks.debug_winners()) == 4
    assert calls["stock"] == 4


def test_channels_last_is_part_of_the_key(timings):
    timings({"native.a": 1.0, "stock": 4.0})
    x, w, s, p, d = args()
    k1 = ks._key("conv2d", x, w, s, p, d)
    k2 = ks._key("conv2d", x.to(memory_format=torch.channels_last), w, s, p, d)
    assert k1 != k2 and k1[:-1] == k2[:-1]


def test_decliner_loses(timings):
    timings({"native.a": 0.1, "stock": 4.0})
    x, w, s, p, d = args()
    assert ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"], declines={"native.a"})) == "out:stock"
    assert list(ks.debug_winners().values()) == ["stock"]


def test_cached_winner_that_declines_is_evicted_and_remeasured(timings):
    calls = timings({"native.a": 1.0, "native.b": 2.0, "stock": 4.0})
    x, w, s, p, d = args()
    ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "native.b", "stock"]))
    assert ks.cached("conv2d", x, w, s, p, d) == "native.a"
    out = ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "native.b", "stock"], declines={"native.a"}))
    assert out == "out:native.b"
    assert ks.cached("conv2d", x, w, s, p, d) == "native.b"
    assert calls["native.b"] == 2


def test_all_decline_returns_none(timings):
    timings({})
    x, w, s, p, d = args()
    assert ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"], declines={"native.a", "stock"})) is None


def test_kill_switch(monkeypatch, timings):
    calls = timings({"native.a": 1.0, "stock": 4.0})
    monkeypatch.setattr(ks, "_ENABLED", False)
    x, w, s, p, d = args()
    assert ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"])) is None
    assert ks.pick_key("group_norm", (1,), cands(["native.a", "stock"])) is None
    assert ks.cached("conv2d", x, w, s, p, d) is None
    assert calls == {}


def test_reset_forgets(timings):
    calls = timings({"native.a": 1.0, "stock": 4.0})
    x, w, s, p, d = args()
    ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"]))
    ks.reset()
    assert ks.debug_winners() == {}
    ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"]))
    assert calls["native.a"] == 2


def test_pick_key_group_norm(timings):
    timings({"native.res": 1.0, "stock": 2.0})
    key = (torch.float16, (8, 512, 64, 64), 32, False)
    assert ks.pick_key("group_norm", key, cands(["native.res", "stock"])) == "out:native.res"
    assert ks.cached_key("group_norm", key) == "native.res"
    assert ks.cached_key("group_norm", (torch.float16, (8, 512, 64, 64), 16, False)) is None


# ---------------------------------------------------------------------------
# verification with real tensors
# ---------------------------------------------------------------------------
def _outs(ref, **others):
    d = {"stock": ref}
    d.update(others)
    return d


def test_wrong_fastest_candidate_is_blacklisted(monkeypatch, timings):
    monkeypatch.setattr(ks, "_VERIFY_ENABLED", True)
    timings({"native.bad": 0.5, "native.good": 1.0, "stock": 3.0})
    ref = torch.randn(4, 64)
    outs = _outs(ref, **{"native.bad": ref + 1.0, "native.good": ref + 1e-6})
    x, w, s, p, d = args()
    with pytest.warns(UserWarning, match="native.bad"):
        out = ks.pick("conv2d", x, w, s, p, d, cands(["native.bad", "native.good", "stock"], outputs=outs))
    assert out is outs["native.good"]
    key = ks._key("conv2d", x, w, s, p, d)
    assert ks.debug_bad_candidates() == {key: {"native.bad"}}
    assert ks.debug_winners()[key] == "native.good"


def test_everything_wrong_falls_back_to_reference(monkeypatch, timings):
    monkeypatch.setattr(ks, "_VERIFY_ENABLED", True)
    timings({"native.a": 0.5, "stock": 3.0})
    ref = torch.randn(8, 8)
    outs = _outs(ref, **{"native.a": -ref})
    x, w, s, p, d = args()
    with pytest.warns(UserWarning):
        out = ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"], outputs=outs))
    assert out is ref
    assert list(ks.debug_winners().values()) == ["stock"]


def test_blacklisted_candidate_never_timed_again(monkeypatch, timings):
    monkeypatch.setattr(ks, "_VERIFY_ENABLED", True)
    calls = timings({"native.a": 0.5, "stock": 3.0})
    ref = torch.randn(8, 8)
    outs = _outs(ref, **{"native.a": ref * 2})
    x, w, s, p, d = args()
    with pytest.warns(UserWarning):
        ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"], outputs=outs))
    with ks._lock:
        ks._winners.clear()
    ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"], outputs=outs))
    assert calls["native.a"] == 1


def test_rms_scaled_bar():
    """Near-zero elements of a large output may disagree by rounding (passes); a dropped
    channel (an order of RMS/sqrt(C) wrong) must fail."""
    torch.manual_seed(0)
    ref = torch.randn(64, 256) * 50.0
    cand = ref.clone()
    small = ref.abs() < 0.05
    cand[small] += 0.002                      # 200x atol 1e-5, below rtol * RMS = 5e-3
    assert ks._verify(cand, ref, (1e-4, 1e-5))
    dropped = ref.clone()
    dropped[:, 3] = 0.0
    assert ks._verify(dropped, ref, (1e-2, 1e-2)) is False
    assert ks._verify(torch.zeros(3), torch.zeros(4)) is False       # shape mismatch
    assert ks._verify(ref.half(), ref.half())


def test_verify_is_chunked(monkeypatch):
    monkeypatch.setattr(ks, "_VERIFY_CHUNK_ELEMENTS", 16)
    ref = torch.randn(40, 8)
    bad = ref.clone()
    bad[37, 5] += 100
    assert ks._verify(ref.clone(), ref) is True
    assert ks._verify(bad, ref) is False


def test_oom_while_verifying_is_indeterminate(monkeypatch, timings):
    monkeypatch.setattr(ks, "_VERIFY_ENABLED", True)
    timings({"native.a": 0.5, "stock": 3.0})
    ref = torch.randn(8, 8)
    outs = _outs(ref, **{"native.a": ref.clone()})

    def boom(*a, **k):
        raise torch.OutOfMemoryError("HIP out of memory")
    monkeypatch.setattr(ks, "_block_disagrees", boom)
    x, w, s, p, d = args()
    with pytest.warns(UserWarning, match="out of memory"):
        out = ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"], outputs=outs))
    assert out is ref
    assert ks.debug_winners() == {} and ks.debug_bad_candidates() == {}


def test_oom_in_candidate_declines_but_other_errors_propagate(monkeypatch, timings):
    timings({"native.a": 0.5, "stock": 3.0})
    x, w, s, p, d = args()

    def oom():
        raise torch.OutOfMemoryError("out of memory")
    oom._name = "native.a"
    monkeypatch.setattr(ks, "_time", lambda fn: {"native.a": 0.5, "stock": 3.0}[fn._name])
    stock = cands(["stock"])[0]
    assert ks.pick("conv2d", x, w, s, p, d, [("native.a", oom), stock]) == "out:stock"
    ks.reset()

    def bug():
        raise RuntimeError("index out of range")
    bug._name = "native.a"
    with pytest.raises(RuntimeError, match="index out of range"):
        ks.pick("conv2d", x, w, s, p, d, [("native.a", bug), stock])


def test_runoff_reranks_close_finishers_by_interleaved_median(monkeypatch, timings):
    """Candidates within the runoff band of the fastest are re-timed together and the
    median order wins; a candidate outside the band is not re-timed."""
    timings({"native.a": 1.00, "native.b": 1.03, "native.c": 1.50, "stock": 3.0})
    seen = []

    def fake_interleaved(fns):
        seen.append([f._name for f in fns])
        return [{"native.a": 1.2, "native.b": 1.1}[f._name] for f in fns]
    monkeypatch.setattr(ks, "_time_interleaved", fake_interleaved)
    x, w, s, p, d = args()
    out = ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "native.b", "native.c", "stock"]))
    assert out == "out:native.b"
    assert seen == [["native.a", "native.b"]]


def test_runoff_keeps_first_round_order_when_retiming_fails(monkeypatch, timings):
    timings({"native.a": 1.00, "native.b": 1.01, "stock": 3.0})
    monkeypatch.setattr(ks, "_time_interleaved", lambda fns: None)
    x, w, s, p, d = args()
    assert ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "native.b", "stock"])) == "out:native.a"


def test_time_reports_none_for_decliners_and_errors():
    assert ks._time(lambda: None) is None

    def err():
        raise RuntimeError("launch failed")
    assert ks._time(err) is None


# ---------------------------------------------------------------------------
# disk cache
# ---------------------------------------------------------------------------
def test_disk_cache_roundtrip_and_versioning(monkeypatch, timings, tmp_path):
    monkeypatch.setattr(ks, "_DISK_CACHE_ENABLED", True)
    monkeypatch.setattr(ks, "_VERIFY_ENABLED", True)
    timings({"native.a": 0.5, "native.b": 1.0, "stock": 3.0})
    ref = torch.randn(8, 8)
    outs = _outs(ref, **{"native.a": ref * 3, "native.b": ref.clone()})
    x, w, s, p, d = args()
    with pytest.warns(UserWarning):
        ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "native.b", "stock"], outputs=outs))
    path = ks._cache_path()
    raw = json.load(open(path))
    assert raw["verify_bar"] == ks._VERIFY_BAR_VERSION
    assert list(raw["winners"].values()) == ["native.b"]
    assert list(raw["bad"].values()) == [["native.a"]]
    key = ks._key("conv2d", x, w, s, p, d)
    assert ks._decode_key(next(iter(raw["winners"]))) == key
    # a fresh process (cleared memory) reloads both sections
    with ks._lock:
        ks._winners.clear()
        ks._bad_candidates.clear()
    monkeypatch.setattr(ks, "_disk_loaded", False)
    assert ks.cached("conv2d", x, w, s, p, d) == "native.b"
    assert ks.debug_bad_candidates() == {key: {"native.a"}}
    # an older verification bar: blacklist AND its shape's winner are dropped
    raw["verify_bar"] = ks._VERIFY_BAR_VERSION - 1
    json.dump(raw, open(path, "w"))
    with ks._lock:
        ks._winners.clear()
        ks._bad_candidates.clear()
    monkeypatch.setattr(ks, "_disk_loaded", False)
    assert ks.cached("conv2d", x, w, s, p, d) is None
    assert ks.debug_bad_candidates() == {}


def test_disk_cache_flat_legacy_format_and_corrupt_file(monkeypatch, tmp_path):
    monkeypatch.setattr(ks, "_DISK_CACHE_ENABLED", True)
    key = ("group_norm", torch.float16, (2, 4), 2, False)
    json.dump({ks._key_str(key): "stock"}, open(ks._cache_path(), "w"))
    monkeypatch.setattr(ks, "_disk_loaded", False)
    assert ks.cached_key("group_norm", key[1:]) == "stock"
    open(ks._cache_path(), "w").write("{not json")
    with ks._lock:
        ks._winners.clear()
    monkeypatch.setattr(ks, "_disk_loaded", False)
    assert ks.cached_key("group_norm", key[1:]) is None      # corrupt file: empty cache, no error


def test_reset_removes_the_file(monkeypatch, timings):
    monkeypatch.setattr(ks, "_DISK_CACHE_ENABLED", True)
    timings({"native.a": 0.5, "stock": 3.0})
    x, w, s, p, d = args()
    ks.pick("conv2d", x, w, s, p, d, cands(["native.a", "stock"]))
    import os
    assert os.path.exists(ks._cache_path())
    ks.reset()
    assert not os.path.exists(ks._cache_path())
