"""Per-shape benchmark-once selection among candidate implementations, stock included.

Behavioural restatement of the reference's selector (amd_tuned_torch/kernel_select.py:
132-733).  On the first call for a shape key every candidate is timed (2 warm-up calls, then
3 individually event-timed calls, minimum kept -- kernel_select.py:430-431,454-492), the
fastest NON-reference candidate is checked numerically against the reference candidate
(always the LAST entry, stock by convention -- kernel_select.py:554-693), and the verified
winner's NAME is cached in memory and in a JSON file keyed by GPU + torch + Python version
(kernel_select.py:310-423).  Later calls with the same key dispatch straight to the winner.

Candidates here are this package's own gfx950 kernel variants (named "native.<variant>")
plus "stock".  Policies kept from the reference because callers and tests depend on them:

* a thunk returning None declines; a cached winner that declines is evicted (memory and
  disk) and the shape re-contested (kernel_select.py:562-571);
* a candidate that measures fastest but fails verification is excluded for that exact key,
  persisted, with a warning; the next-fastest is verified in turn, down to the reference
  (kernel_select.py:670-680);
* the verification bar is max(atol, rtol * RMS(reference)), compared in 8M-element chunks
  (kernel_select.py:164-295); an OOM while comparing is INDETERMINATE: the reference output
  is served and nothing is recorded (kernel_select.py:652-669);
* an OOM inside a candidate or the reference is a decline, any other exception propagates
  (kernel_select.py:597-629);
* blacklists written under another verification-bar version are dropped together with the
  winners of those keys (kernel_select.py:297-309,378-395);
* AMD_TUNED_TORCH_MEASURE_KERNELS=0 (legacy AMD_TUNED_TORCH_CONV_MEASURE) disables the
  contest, AMD_TUNED_TORCH_KERNEL_SELECT_VERIFY=0 skips verification,
  AMD_TUNED_TORCH_KERNEL_SELECT_CACHE=0 disables the disk file and
  AMD_TUNED_TORCH_KERNEL_SELECT_CACHE_DIR relocates it (all read once at import).
"""
from __future__ import annotations

import contextlib
import json
import math
import os
import re
import sys
import threading
import warnings
from typing import Callable, Optional

import torch

_ENABLED = (os.environ.get("AMD_TUNED_TORCH_MEASURE_KERNELS",
                           os.environ.get("AMD_TUNED_TORCH_CONV_MEASURE", "1")) != "0")
_VERIFY_ENABLED = os.environ.get("AMD_TUNED_TORCH_KERNEL_SELECT_VERIFY", "1") != "0"

_winners: dict = {}          # key -> winning candidate name
_bad_candidates: dict = {}   # key -> {names that failed verification}
_lock = threading.Lock()

# (rtol, atol) per output dtype (kernel_select.py:150-155)
_TOLERANCES = {
    torch.float16: (1e-2, 1e-2),
    torch.bfloat16: (2e-2, 2e-2),
    torch.float32: (1e-4, 1e-5),
}
_DEFAULT_TOLERANCE = (2e-2, 2e-2)

_VERIFY_SCALE_SAMPLE = 1 << 20     # elements sampled (strided) for the RMS scale
_VERIFY_CHUNK_ELEMENTS = 1 << 23   # elements upcast per comparison slice

_VERIFY_BAR_VERSION = 3
_DISK_CACHE_ENABLED = os.environ.get("AMD_TUNED_TORCH_KERNEL_SELECT_CACHE", "1") != "0"
_CACHE_DIR = os.environ.get(
    "AMD_TUNED_TORCH_KERNEL_SELECT_CACHE_DIR",
    os.path.join(os.path.dirname(os.path.abspath(__file__)), "_kernel_select_cache"))

_WARMUP = 2
_ITERS = 3

# Runoff among close finishers: the minimum of _ITERS runs cannot separate kernels a few per
# cent apart, so candidates within _RUNOFF_BAND of the fastest (at most _RUNOFF_MAX of them)
# are re-timed _RUNOFF_ROUNDS times, interleaved, and ranked by their median.
_RUNOFF_BAND = 0.08
_RUNOFF_MAX = 3
_RUNOFF_ROUNDS = 7

# The disk cache is read on first use rather than at import, so importing the package does
# not initialise the GPU runtime (the cache file name embeds the GPU model).
_disk_loaded = False


def _ensure_disk_cache() -> None:
    global _disk_loaded
    if not _disk_loaded:
        _disk_loaded = True
        _load_disk_cache()


def enabled() -> bool:
    return _ENABLED


# ---------------------------------------------------------------------------
# verification
# ---------------------------------------------------------------------------
def _is_oom(exc: BaseException) -> bool:
    for cls in (getattr(torch, "OutOfMemoryError", None),
                getattr(getattr(torch, "cuda", None), "OutOfMemoryError", None)):
        if isinstance(cls, type) and isinstance(exc, cls):
            return True
    return "out of memory" in str(exc).lower()


def _reference_scale(reference_out) -> Optional[float]:
    """RMS of a strided sample of the reference output (None if not measurable)."""
    try:
        flat = reference_out.detach().flatten()
        step = max(1, flat.numel() // _VERIFY_SCALE_SAMPLE)
        rms = float(flat[::step].float().pow(2).mean().sqrt())
    except (RuntimeError, TypeError, ValueError, AttributeError, ZeroDivisionError):
        return None
    return rms if (math.isfinite(rms) and rms > 0.0) else None


def _block_disagrees(cand: torch.Tensor, ref: torch.Tensor, rtol: float, atol: float) -> bool:
    """True if some element of the fp32 block pair is not within atol + rtol * |ref| of the
    reference.  NaN matches only NaN and an infinity only the same infinity (torch.allclose
    with equal_nan semantics)."""
    c, r = cand.float(), ref.float()
    finite = torch.isfinite(c) & torch.isfinite(r)
    off = (c - r).abs_() > r.abs().mul_(rtol).add_(atol)
    if bool((off & finite).any()):
        return True
    odd = ~finite
    if not bool(odd.any()):
        return False
    both_nan = c.isnan() & r.isnan()
    same_inf = torch.isinf(c) & (c == r)
    return bool((odd & ~(both_nan | same_inf)).any())


def _row_blocks(n_rows: int, per_row: int):
    """[lo, hi) ranges of dim-0 rows holding about _VERIFY_CHUNK_ELEMENTS elements each: a
    slice along dim 0 is always a view, so no full-size copy is ever made."""
    rows = max(1, _VERIFY_CHUNK_ELEMENTS // max(1, per_row))
    return ((lo, min(n_rows, lo + rows)) for lo in range(0, n_rows, rows))


def _verify(candidate_out, reference_out, tolerance=None) -> Optional[bool]:
    """Does the candidate's output agree with the reference's?  True / False, or None when the
    comparison itself ran out of memory (no verdict about the kernel).  The bar is the
    reference's (kernel_select.py:164-295): max(atol, rtol * RMS(reference)) absolute plus
    rtol relative, with (rtol, atol) from `tolerance` or the dtype table.  Anything that
    keeps the comparison from running for a reason of the candidate's own (wrong shape, not
    a tensor) is a disagreement."""
    try:
        cand, ref = candidate_out.detach(), reference_out.detach()
        rtol, atol = tolerance or _TOLERANCES.get(cand.dtype, _DEFAULT_TOLERANCE)
        scale = _reference_scale(ref)
        atol = atol if scale is None else max(atol, rtol * scale)
        if cand.shape != ref.shape:
            return False
        if cand.dim() == 0:
            return not _block_disagrees(cand.reshape(1), ref.reshape(1), rtol, atol)
        per_row = cand.numel() // max(1, cand.shape[0])
        return not any(_block_disagrees(cand[lo:hi], ref[lo:hi], rtol, atol)
                       for lo, hi in _row_blocks(cand.shape[0], per_row))
    except (RuntimeError, TypeError, ValueError, AttributeError) as exc:
        return None if _is_oom(exc) else False


# ---------------------------------------------------------------------------
# disk cache
# ---------------------------------------------------------------------------
def _device_key() -> str:
    try:
        name = torch.cuda.get_device_name(0) if torch.cuda.is_available() else "cpu"
    except Exception:
        name = "unknown"
    name = re.sub(r"[^A-Za-z0-9_.-]+", "_", name)
    tv = torch.__version__.replace("+", "_").replace("/", "_")
    return f"{name}-torch-{tv}-cp{sys.version_info.major}{sys.version_info.minor}"


def _cache_path() -> str:
    return os.path.join(_CACHE_DIR, f"{_device_key()}.json")


def _encode(v):
    if isinstance(v, torch.dtype):
        return {"__dtype__": str(v)}
    if isinstance(v, tuple):
        return {"__tuple__": [_encode(e) for e in v]}
    return v


def _decode(v):
    if isinstance(v, dict):
        if "__dtype__" in v:
            return getattr(torch, v["__dtype__"].rsplit(".", 1)[-1])
        if "__tuple__" in v:
            return tuple(_decode(e) for e in v["__tuple__"])
    return v


def _key_str(key) -> str:
    return json.dumps([_encode(e) for e in key])


def _decode_key(s: str):
    return tuple(_decode(e) for e in json.loads(s))


def _file_payload() -> dict:
    """The cache file's content (call with _lock held).  Sections: the verification-bar
    version, winner names and excluded names per encoded key -- the reference's format
    (kernel_select.py:310-423), so either package reads the other's file."""
    return {
        "verify_bar": _VERIFY_BAR_VERSION,
        "winners": {_key_str(k): name for k, name in _winners.items()},
        "bad": {_key_str(k): sorted(names) for k, names in _bad_candidates.items() if names},
    }


def _absorb_payload(raw) -> None:
    """Merge a cache file's content into memory (entries already in memory win).  A flat
    {key: winner} file from before the sections existed is read as winners.  Exclusions
    judged under another verification bar are not evidence under this one: they are
    dropped, and so are the winners of their keys, so those shapes are contested again."""
    if not isinstance(raw, dict):
        return
    sectioned = "winners" in raw or "bad" in raw
    winners = raw.get("winners", {}) if sectioned else raw
    excluded = raw.get("bad", {}) if sectioned else {}
    current = raw.get("verify_bar") == _VERIFY_BAR_VERSION

    def decoded(items):
        for text, value in items:
            try:
                yield _decode_key(text), text, value
            except (ValueError, TypeError, AttributeError):
                continue

    with _lock:
        for key, text, name in decoded(winners.items()):
            if current or text not in excluded:
                _winners.setdefault(key, name)
        if current:
            for key, _, names in decoded(excluded.items()):
                _bad_candidates.setdefault(key, set()).update(names)


def _load_disk_cache() -> None:
    """Read this GPU's cache file, if enabled and readable (a missing or corrupt file is an
    empty cache, never an error)."""
    if not _DISK_CACHE_ENABLED:
        return
    try:
        with open(_cache_path(), "r") as f:
            _absorb_payload(json.load(f))
    except (OSError, ValueError):
        return


def _save_disk_cache() -> None:
    """Write the whole cache file: a per-process temporary file renamed over the old one, so
    readers only ever see a complete file."""
    if not _DISK_CACHE_ENABLED:
        return
    path = _cache_path()
    with _lock:
        payload = _file_payload()
    tmp = f"{path}.tmp{os.getpid()}"
    try:
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(tmp, "w") as f:
            json.dump(payload, f)
        os.replace(tmp, path)
    except OSError:
        pass


# ---------------------------------------------------------------------------
# keys, timing, lookup
# ---------------------------------------------------------------------------
def _norm(v):
    return (v,) if isinstance(v, int) else tuple(v)


def _key(kind, input, weight, stride, padding, dilation):
    # memory format is part of the identity (kernel_select.py:438-445)
    nd = input.dim()
    channels_last = ((nd == 4 and input.is_contiguous(memory_format=torch.channels_last))
                     or (nd == 5 and input.is_contiguous(memory_format=torch.channels_last_3d)))
    return (kind, input.dtype, tuple(input.shape), tuple(weight.shape), _norm(stride),
            _norm(padding), _norm(dilation), channels_last)


# GPU spin queued ahead of the timed runs (clock cycles): long enough for the host to enqueue
# every timed call before the GPU reaches the first event, so each event pair brackets GPU
# time only -- otherwise a kernel shorter than the Python dispatch is timed as the dispatch.
_LEAD_CYCLES = 2_000_000


def _lead(calls: int) -> None:
    """Queue the GPU spin that covers the host's enqueue of `calls` timed calls."""
    if _LEAD_CYCLES and hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(_LEAD_CYCLES * max(1, -(-calls // _ITERS)))


def _time(fn) -> Optional[float]:
    """Minimum over _ITERS individually event-timed runs, after _WARMUP runs; None if the
    candidate declines or raises a Runtime/Type/AssertionError."""
    try:
        for _ in range(_WARMUP):
            if fn() is None:
                return None
        torch.cuda.synchronize()
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(_ITERS)]
        _lead(_ITERS)
        for a, b in pairs:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return min(a.elapsed_time(b) for a, b in pairs)
    except (RuntimeError, TypeError, AssertionError):
        return None


def _time_interleaved(fns) -> Optional[list]:
    """Median event-timed duration of each fn over _RUNOFF_ROUNDS rounds that run every fn
    once in turn (so clock and thermal drift hit all alike); None on any error."""
    if not torch.cuda.is_available():
        return None
    try:
        events = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in fns] for _ in range(_RUNOFF_ROUNDS)]
        torch.cuda.synchronize()
        _lead(len(fns) * _RUNOFF_ROUNDS)
        for row in events:
            for fn, (a, b) in zip(fns, row):
                a.record()
                fn()
                b.record()
        torch.cuda.synchronize()
        meds = []
        for j in range(len(fns)):
            ts = sorted(row[j][0].elapsed_time(row[j][1]) for row in events)
            meds.append(ts[len(ts) // 2])
        return meds
    except (RuntimeError, TypeError, AssertionError):
        return None


def _runoff(timed: list) -> list:
    """Re-rank the close finishers of a sorted [(ms, name, thunk)] list by _time_interleaved."""
    if len(timed) < 2:
        return timed
    best = timed[0][0]
    close = [r for r in timed[:_RUNOFF_MAX] if r[0] <= best * (1.0 + _RUNOFF_BAND)]
    if len(close) < 2:
        return timed
    meds = _time_interleaved([thunk for _, _, thunk in close])
    if meds is None:
        return timed
    ranked = sorted(((m, name, thunk) for m, (_, name, thunk) in zip(meds, close)),
                    key=lambda r: r[0])
    return ranked + timed[len(close):]


def cached(kind: str, input, weight, stride, padding, dilation) -> Optional[str]:
    """Winner already decided for this conv shape, or None."""
    if not _ENABLED:
        return None
    _ensure_disk_cache()
    key = _key(kind, input, weight, stride, padding, dilation)
    with _lock:
        return _winners.get(key)


def cached_key(kind: str, key) -> Optional[str]:
    if not _ENABLED:
        return None
    _ensure_disk_cache()
    with _lock:
        return _winners.get((kind,) + tuple(key))


def pick(kind: str, input, weight, stride, padding, dilation,
         candidates: "list[tuple[str, Callable]]", tolerance=None):
    """Output of the fastest verified candidate for this conv shape (None when disabled).
    The last candidate is the reference (stock) and is assumed to always work."""
    if not _ENABLED:
        return None
    return _contest(_key(kind, input, weight, stride, padding, dilation), candidates, tolerance)


def pick_key(kind: str, key, candidates: "list[tuple[str, Callable]]", tolerance=None):
    """Same as pick() over a caller-built key (group_norm keys on the group count)."""
    if not _ENABLED:
        return None
    return _contest((kind,) + tuple(key), candidates, tolerance)


def _record(key, name: str) -> None:
    with _lock:
        _winners[key] = name
    _save_disk_cache()


def _call_guarded(thunk):
    """Run a thunk; an OOM becomes (None, True), other Runtime/Type/AssertionErrors raise."""
    try:
        return thunk(), False
    except (RuntimeError, TypeError, AssertionError) as exc:
        if not _is_oom(exc):
            raise
        return None, True


def _contest(key, candidates, tolerance=None):
    if not candidates:
        return None
    _ensure_disk_cache()
    ref_name, ref_thunk = candidates[-1]
    with _lock:
        winner = _winners.get(key)
        bad = set(_bad_candidates.get(key, ()))

    if winner is not None and winner not in bad:
        for name, thunk in candidates:
            if name == winner:
                out = thunk()
                if out is not None:
                    return out
                break
        with _lock:  # cached winner declined (or is no longer offered): evict, re-contest
            _winners.pop(key, None)
        _save_disk_cache()

    timed = []
    for name, thunk in candidates:
        if name in bad:
            continue
        ms = _time(thunk)
        if ms is not None:
            timed.append((ms, name, thunk))
    timed.sort(key=lambda r: r[0])
    timed = _runoff(timed)

    ref_out = None
    ref_done = False
    ref_oom = False
    for _, name, thunk in timed:
        out, _oom = _call_guarded(thunk)
        if out is None:
            continue
        if name == ref_name or not _VERIFY_ENABLED:
            _record(key, name)
            return out
        if not ref_done:
            ref_done = True
            ref_out, ref_oom = _call_guarded(ref_thunk)
            if ref_out is None:
                if ref_oom:
                    return out          # nothing learned: serve, record nothing
                _record(key, name)      # reference declined: nothing to verify against
                return out
        verdict = _verify(out, ref_out, tolerance)
        if verdict:
            _record(key, name)
            return out
        if verdict is None:
            warnings.warn(
                f"amd_tuned_torch.kernel_select: ran out of memory verifying candidate "
                f"'{name}' for {key} against '{ref_name}'; serving the reference for this "
                "call and recording nothing (not evidence that the candidate is wrong).",
                UserWarning)
            return ref_out
        warnings.warn(
            f"amd_tuned_torch.kernel_select: candidate '{name}' for {key} measured fastest but "
            f"did not match '{ref_name}' within tolerance; excluding it for this exact shape.",
            UserWarning)
        with _lock:
            _bad_candidates.setdefault(key, set()).add(name)
        _save_disk_cache()

    if ref_oom:
        return ref_out
    if ref_done and ref_out is not None:
        _record(key, ref_name)
        return ref_out
    return None


def debug_winners() -> dict:
    """{key: winning candidate name}."""
    _ensure_disk_cache()
    with _lock:
        return dict(_winners)


def debug_bad_candidates() -> dict:
    """{key: {names excluded for failing verification}}."""
    with _lock:
        return {k: set(v) for k, v in _bad_candidates.items()}


def reset() -> None:
    """Forget every winner and exclusion, in memory and in this GPU's cache file."""
    global _disk_loaded
    with _lock:
        _winners.clear()
        _bad_candidates.clear()
    _disk_loaded = True  # the file is gone too: nothing to merge back in later
    if _DISK_CACHE_ENABLED:
        with contextlib.suppress(OSError):
            os.remove(_cache_path())
