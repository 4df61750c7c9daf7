"""HipFallbackWarning bookkeeping (CPU): a torch fallback warns once per function and reason under the default
filter, and raises on every call when the caller turns the warning into an error."""

from __future__ import annotations

import warnings

import pytest

from hclsm_amd.kernels import HipFallbackWarning, _common


def test_warns_once_per_reason():
    _common._WARNED.clear()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        _common.warn_fallback("probe_fn", "reason a")
        _common.warn_fallback("probe_fn", "reason a")
        _common.warn_fallback("probe_fn", "reason b")
    msgs = [str(w.message) for w in rec if issubclass(w.category, HipFallbackWarning)]
    assert len(msgs) == 2 and "reason a" in msgs[0] and "reason b" in msgs[1]
    _common._WARNED.clear()


def test_error_filter_raises_on_every_call():
    _common._WARNED.clear()
    with warnings.catch_warnings():
        warnings.simplefilter("error", HipFallbackWarning)
        for _ in range(3):
            with pytest.raises(HipFallbackWarning):
                _common.warn_fallback("probe_fn", "reason a")
    _common._WARNED.clear()
