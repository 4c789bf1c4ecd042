"""The C ABI loads and exports every symbol include/jitcast_hip.h declares; host-side helpers and
error paths that need no GPU (CPU only)."""
import ctypes

import numpy as np
import pytest

from jitcast_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _lib.header_symbols()
    assert declared, "no declarations parsed"
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # the Python binding types every declared function
    assert sorted(_lib.SIGNATURES) == declared


def test_rope_table_matches_oracle_bit_exact(oracle):
    from jitcast_amd import chronos2

    for n, dh in ((513, 64), (37, 64), (20, 16), (9, 48)):
        np.testing.assert_array_equal(chronos2.rope_table(n, dh), oracle.c2_rope_table(n, dh))


def test_rope_table_rejects_bad_arguments():
    buf = np.empty(16, np.float32)
    with pytest.raises(_lib.JitcastArgumentError, match="jc_c2_rope_table"):
        _lib.call("jc_c2_rope_table", 4, 3, ctypes.c_float(1e4), buf.ctypes.data_as(ctypes.c_void_p))


def test_null_context_is_an_error_not_a_crash():
    rc = _lib.lib().jc_c2_time_attention(None, None, None, None, None, 1, 1, 1, 64, 64, 0)
    assert rc == _lib.JC_EINVAL
    assert "null context" in _lib.last_error()
    assert _lib.lib().jc_sync(None) == _lib.JC_EINVAL


def test_version():
    assert _lib.lib().jc_version() >= 1


def test_static_layer_scratch_size_matches_header():
    """The Python binding's LAYER_STATIC_BYTES is the header's JC_C2_LAYER_STATIC_BYTES."""
    import re

    from jitcast_amd import chronos2

    text = _lib.HEADER.read_text()
    m = re.search(r"#define JC_C2_LAYER_STATIC_BYTES \((\d+)u << (\d+)\)", text)
    assert m, "JC_C2_LAYER_STATIC_BYTES not found"
    assert chronos2.LAYER_STATIC_BYTES == int(m.group(1)) << int(m.group(2))


def test_static_layer_null_context_is_an_error():
    rc = _lib.lib().jc_c2_layer_static(None, None, None, None, None, None, None, 1, 1, 64, 1, 64, 64,
                                       ctypes.c_float(1e-6), 0)
    assert rc == _lib.JC_EINVAL
    assert "null context" in _lib.last_error()
