"""The C-ABI library loads on a CPU-only host and exports every symbol that
include/kadconv_hip.h declares (no compute calls without a GPU)."""
import ctypes
import os
import re

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, 'include', 'kadconv_hip.h')


def _declared():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(kad_[a-z0-9_]+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    from kadconv import _ext
    lib = ctypes.CDLL(_ext.lib_path())
    names = _declared()
    assert 'kad_dcn_fwd' in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    from kadconv import _ext
    assert set(_declared()) == set(_ext.SIGNATURES), set(_declared()) ^ set(_ext.SIGNATURES)


def test_pure_host_entry_points():
    from kadconv import _ext
    lib = _ext.load()
    assert lib.kad_abi_version() == _ext.ABI_VERSION
    assert lib.kad_dcn_wpack_elems(86, 86) == 96 * 3 * 9 * 32
    t = lib.kad_dcn_tiles(100, 100)
    assert 10000 / 128 <= t <= 10000 / 64  # tiles hold at most 128 pixels and waste little
    # argument validation happens before any device work
    assert lib.kad_dcn_fwd(None, None) < 0
    assert b'null' in lib.kad_last_error()


def test_se_nchw_fits_rule():
    """kad_se_nchw_fits: the two-launch NCHW SE takes C % 32 == 0, 1 <= hidden <= 64 and planes of
    at least 8 pixels (a 16-byte piece meets at most two planes); other shapes keep the
    pool / MLP / scale launches.  kad_se_nchw itself rejects a shape that does not fit."""
    from kadconv import _ext
    lib = _ext.load()
    assert lib.kad_se_nchw_fits(16, 1024, 25, 25, 64) == 1
    assert lib.kad_se_nchw_fits(1, 32, 1, 8, 1) == 1
    assert lib.kad_se_nchw_fits(2, 48, 7, 9, 3) == 0     # C % 32 != 0
    assert lib.kad_se_nchw_fits(1, 32, 1, 7, 4) == 0     # 7-pixel planes
    assert lib.kad_se_nchw_fits(1, 64, 8, 8, 65) == 0    # hidden > 64
    assert lib.kad_se_nchw_fits(0, 64, 8, 8, 4) == 0
    assert lib.kad_se_nchw(None, None, None, None, None, None, None, None, 1, 64, 8, 8, 4, _ext.KAD_F16, None) < 0
    assert b'null' in lib.kad_last_error()
