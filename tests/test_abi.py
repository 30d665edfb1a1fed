"""The C-ABI library: builds, loads without a GPU, exports every symbol the
public header declares, and fails cleanly (status codes, no crash) where no
device is needed to tell.  CPU only."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from conftest import ROOT, gpu_available

HEADER = ROOT / "include" / "pagellm_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(plh_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from pagellm_amd import _native

    if not _native.LIB_PATH.exists():
        from pagellm_amd.build import build

        build()
    return _native.load_library()


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ["plh_sample", "plh_verify", "plh_draw", "plh_penalize", "plh_create", "plh_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_signatures_cover_the_header(lib):
    from pagellm_amd import _native

    assert sorted(_native.SIGNATURES) == _declared()


def test_abi_version_matches_header(lib):
    m = re.search(r"#define PLH_ABI_VERSION (\d+)", HEADER.read_text())
    assert lib.plh_abi_version() == int(m.group(1))


def test_status_codes_match_header():
    from pagellm_amd import _native

    text = HEADER.read_text()
    for name in ["PLH_OK", "PLH_ERR_INVALID_ARG", "PLH_ERR_HIP", "PLH_ERR_OUT_OF_MEMORY", "PLH_ERR_UNSUPPORTED",
                 "PLH_ERR_NO_DEVICE", "PLH_F32", "PLH_F64", "PLH_SAMPLE_ROWWISE", "PLH_SAMPLE_HIST_SPANS", "PLH_SAMPLE_NUCLEUS",
                 "PLH_SAMPLE_NUCLEUS_ONLY", "PLH_OPT_KERNEL_TIMING"]:
        m = re.search(rf"#define {name} (-?\d+)", text)
        assert m and int(m.group(1)) == getattr(_native, name), name


def test_null_context_is_an_invalid_argument(lib):
    assert lib.plh_sample(None, None, 0, 1, 1, 1, None, None, None, None, None, None, None, None, None, 0) == -1
    assert lib.plh_verify(None, None, None, 0, 1, 1, 1, None, None, None, 0, None, None) == -1
    assert lib.plh_draw(None, None, 0, 1, 1, 1, None, None) == -1
    assert lib.plh_penalize(None, None, 0, 1, 1, 1, None, None, None, None, 1) == -1
    assert lib.plh_sync(None) == -1
    assert lib.plh_set_option(None, 1, 1) == -1
    assert lib.plh_kernel_times(None, None, None, None) == -1
    assert lib.plh_append_ids(None, None, None, None, 1) == -1
    assert lib.plh_copy_rows(None, None, 8, None, 8, 8, 1) == -1
    assert lib.plh_rmsnorm_lm_head(None, None, 4, 1, 4, None, 1e-5, None, 4, 4, None, 4) == -1
    assert lib.plh_host_alloc(None, None, 8) == -1
    assert lib.plh_host_free(None, None) == -1
    assert lib.plh_h2d_async(None, None, None, 8) == -1
    assert lib.plh_last_error(None) == b"null context"
    lib.plh_destroy(None)


@pytest.mark.skipif(gpu_available(), reason="checks the no-device status code")
def test_create_without_device_reports_no_device(lib):
    h = ctypes.c_void_p()
    assert lib.plh_create(ctypes.byref(h), 0) == -5
    assert h.value is None


@pytest.mark.skipif(gpu_available(), reason="checks the no-device behaviour")
def test_compute_without_device_raises():
    import numpy as np

    from pagellm_amd import _native
    from pagellm_amd.sampling import SamplingParams, sample

    _native._default = None
    with pytest.raises(_native.PLHError):
        sample(np.zeros(4, dtype=np.float32), SamplingParams(temperature=0), None)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from pagellm_amd import _native

    monkeypatch.setattr(_native, "LIB_PATH", Path(tmp_path) / "libpagellm_hip.so")
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(ImportError):
        _native.load_library()
