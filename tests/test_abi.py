"""The C-ABI library: it builds, loads without a GPU, exports every entry point
include/koptim.h declares, and rejects bad arguments on the host (no compute
calls here)."""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "koptim.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(?:int|long long)\s+(ko_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def libpath():
    import kernel_optim_amd.build as B
    if not os.path.exists(B.LIB_PATH):
        B.build()
    return B.LIB_PATH


def test_header_declares_entry_points():
    names = declared()
    assert "ko_decode_attn" in names and len(names) >= 3


def test_library_exports_every_declared_symbol(libpath):
    out = subprocess.run(["nm", "-D", "--defined-only", libpath], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\sT\s+(ko_\w+)", out))
    missing = [n for n in declared() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_binding_covers_header(libpath):
    from kernel_optim_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared()
    h = _lib.lib()
    for name in declared():
        assert isinstance(getattr(h, name), ctypes._CFuncPtr)


def test_host_side_argument_errors_without_gpu(libpath):
    """Null pointers / unsupported shapes are refused before any launch, so these
    calls are safe on a machine without a GPU."""
    from kernel_optim_amd import _lib
    h = _lib.lib()
    st = h.ko_decode_attn_partial(None, None, None, None, 1, 64, 0, 0, 1, 1, 8, 128, 64, 1, 1,
                                  0.1, None, None, None)
    assert st == -22
    fake = 1 << 20  # never dereferenced: the shape check fails first
    st = h.ko_decode_attn_partial(fake, fake, fake, fake, 1, 64, 0, 0, 1, 1, 8, 64, 64, 1, 1,
                                  0.1, fake, fake, None)
    assert st == -95
    st = h.ko_decode_attn_partial(fake, fake, fake, fake, 1, 64, 0, 0, 1, 1, 8, 128, 64, 0, 1,
                                  0.1, fake, fake, None)
    assert st == -34


def test_wrapper_raises_runtime_error_on_status():
    from kernel_optim_amd import _lib
    assert "invalid argument" in _lib.status_message(-22)
    with pytest.raises(RuntimeError):
        _lib.call("ko_decode_attn_partial", None, None, None, None, 1, 64, 0, 0, 1, 1, 8, 128,
                  64, 1, 1, 0.1, None, None, None)


def test_gemv_host_path_of_every_layout_without_gpu(libpath):
    """ko_gemv's host logic for every layout runs to the launch without a fault
    (layout 3 once divided by the layout-1 wave count, zero there); with no GPU
    the launch itself reports a HIP status. Bad layout-1 wave counts are refused
    first. Skipped where a GPU is visible: the pointers are fake."""
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("fake pointers must not reach a real launch")
    from kernel_optim_amd import _lib
    h = _lib.lib()
    P = 1 << 20
    for K, layout, rows, waves in [(4096, 3, 4, 0), (4096, 3, 8, 0), (9728, 3, 4, 0),
                                   (9728, 3, 19, 0), (2560, 3, 1, 0), (2560, 2, 1, 0),
                                   (2560, 0, 8, 0), (9728, 4, 10, 0), (4096, 4, 10, 0)]:
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, 2, 2560, K,
                       1, 0, 0, layout, rows, waves, 1e-6, None)
        assert st > 0, (K, layout, rows, st)   # a HIP status from the launch, not a host error
    for waves in (0, 1, 3):
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, 2, 2560,
                       2560, 1, 0, 0, 1, 2, waves, 1e-6, None)
        assert st == -95
    st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 16, 2, 2560, 4096, 1, 0,
                   0, 3, 4, 0, 1e-6, None)
    assert st == -34   # layout 3 scratch too small
    st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 16, 2, 2560, 4096, 1, 0,
                   0, 4, 10, 0, 1e-6, None)
    assert st == -34   # layout 4 scratch too small
    for K, norm, rows in [(2560, 1, 10), (4096, 0, 8), (2560 + 512, 0, 10)]:
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, 2, 2560, K,
                       1, norm, 0, 4, rows, 0, 1e-6, None)
        assert st == -95, (K, norm, rows, st)   # layout 4: no NORM, 10 waves, K = 512 S
    assert h.ko_gemv_argmax_scratch(2560, 4, 10, 0) == 192 + 160 * 3 * 256
    # layout 2 with two row tiles (waves 2): 32 rows per launch slice, K in {2560, 4096}
    for M, K, epi in [(20, 2560, 0), (40, 2560, 3), (32, 4096, 2)]:
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, M, 2560, K,
                       epi, 0, 0, 2, 1, 2, 1e-6, None)
        assert st > 0, (M, K, epi, st)
    for K, epi, waves in [(9728, 1, 2), (4096, 3, 2), (2560, 1, 1), (2560, 1, 4)]:
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, 20, 2560, K,
                       epi, 0, 0, 2, 1, waves, 1e-6, None)
        assert st == -95, (K, epi, waves, st)
    # layout 4 with two row tiles: scratch slots of 32 x 16 floats
    for M, K in [(20, 9728), (40, 4096), (32, 2560)]:
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, M, 2560, K,
                       1, 0, 0, 4, 10, 2, 1e-6, None)
        assert st > 0, (M, K, st)
    st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, 20, 2560, 9728,
                   1, 0, 0, 4, 10, 1, 1e-6, None)
    assert st == -95
    st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P,
                   192 + 160 * 3 * 256, 20, 2560, 9728, 1, 0, 0, 4, 10, 2, 1e-6, None)
    assert st == -34   # the one-tile scratch is too small for two tiles
    assert h.ko_gemv_argmax_scratch(2560, 4, 10, 2) == 192 + 160 * 3 * 512
    # four row tiles: 64 rows per launch slice, slots of 64 x 16 floats
    for M in (40, 64, 100):
        st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, M, 2560,
                       9728, 1, 0, 0, 4, 10, 4, 1e-6, None)
        assert st > 0, (M, st)
    st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P,
                   192 + 160 * 3 * 512, 40, 2560, 9728, 1, 0, 0, 4, 10, 4, 1e-6, None)
    assert st == -34
    assert h.ko_gemv_argmax_scratch(2560, 4, 10, 4) == 192 + 160 * 3 * 1024
    st = h.ko_gemv(P, P, P, P, None, P, None, None, None, None, None, P, 1 << 30, 40, 2560, 9728,
                   1, 0, 0, 4, 10, 3, 1e-6, None)
    assert st == -95
    # ARGMAX partials: 160 tiles on 160 workgroups, 16 or 32 rows each
    assert h.ko_gemv_argmax_scratch(2560, 2, 1, 0) == 2 * 16 * 160
    assert h.ko_gemv_argmax_scratch(2560, 2, 1, 2) == 2 * 32 * 160
