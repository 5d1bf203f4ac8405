"""The profile tools of bench.py on synthetic rocprofv3 CSVs (CPU only): the
kernel-trace summary (--trace-md), the dominant kernel's HBM bytes from the two
--pmc runs (--traffic-from) and the per-kernel counter table (--counters-from).
Each expected figure is worked out by hand from the rows below."""
import csv

import pytest

import bench

TRACE_COLS = ['Kernel_Name', 'Grid_Size_X', 'Grid_Size_Y', 'Grid_Size_Z', 'Workgroup_Size_X', 'VGPR_Count',
              'Accum_VGPR_Count', 'LDS_Block_Size', 'Start_Timestamp', 'End_Timestamp']
PMC_COLS = ['Kernel_Name', 'Grid_Size', 'Counter_Name', 'Counter_Value']
COPY = '__amd_rocclr_copyBuffer'


def _write(path, cols, rows):
    with open(path, 'w', newline='') as f:
        w = csv.writer(f)
        w.writerow(cols)
        w.writerows(rows)
    return str(path)


def test_trace_md(tmp_path, capsys):
    # kA: three dispatches of 10, 12 and 8 us (timestamps in ns); kB: one of 1 us
    trace = _write(tmp_path / 't.csv', TRACE_COLS, [
        ['kA', 256, 1, 1, 256, 64, 0, 1024, 0, 10000],
        ['kA', 256, 1, 1, 256, 64, 0, 1024, 20000, 32000],
        ['kA', 256, 1, 1, 256, 64, 0, 1024, 40000, 48000],
        ['kB', 512, 2, 1, 64, 32, 0, 0, 50000, 51000]])
    bench.trace_md(trace, 'Title', 'the command', 'A description.')
    out = capsys.readouterr().out.splitlines()
    assert out[0] == '# Title' and 'the command' in out and 'A description.' in out
    rows = [line for line in out if line.startswith('| `')]
    assert rows[0] == '| `kA` | (256, 1, 1) | 256 | 64 | 0 | 1024 | 3 | 10.00 | 10.00 | 96.8 |'
    assert rows[1] == '| `kB` | (512, 2, 1) | 64 | 32 | 0 | 0 | 1 | 1.00 | 1.00 | 3.2 |'


def test_traffic_from(tmp_path, monkeypatch):
    # the 64 MiB copy reads as 32768 KiB fetched (scale 2) and 65536 KiB written (scale 1)
    dsc = '_ZN3kad14dcn_fwd_kernelIDF16_DF16_Li6ELi1EEEv12kad_dcn_argsNS_7DcnGeomE'
    fetch = _write(tmp_path / 'f.csv', PMC_COLS, [[COPY, 131072, 'FETCH_SIZE', 32768.0]] * 3 +
                   [[dsc, 327680, 'FETCH_SIZE', 10000.0]] * 2 + [[dsc, 4096, 'FETCH_SIZE', 1.0]])
    write = _write(tmp_path / 'w.csv', PMC_COLS, [[COPY, 131072, 'WRITE_SIZE', 65536.0]] * 3 +
                   [[dsc, 327680, 'WRITE_SIZE', 15000.0]] * 2)
    monkeypatch.setattr(bench, 'TRAFFIC_FILE', str(tmp_path / 'traffic.json'))
    bench.traffic_from(fetch, write)
    import json
    out = json.load(open(tmp_path / 'traffic.json'))
    assert out['fetch_scale'] == pytest.approx(2.0) and out['write_scale'] == pytest.approx(1.0)
    # the largest grid of the kernel is the one measured: 10000 KiB x 2 read, 15000 KiB written
    assert out['read_bytes'] == pytest.approx(10000 * 1024 * 2)
    assert out['write_bytes'] == pytest.approx(15000 * 1024)
    assert out['bytes_per_launch'] == pytest.approx(35.84e6, rel=1e-3)


def test_counters_from(tmp_path):
    k = '_ZN3kad5k_fooE'
    trace = _write(tmp_path / 't.csv', TRACE_COLS, [[k, 1024, 1, 1, 256, 8, 0, 0, 0, 10000]] * 3 +
                   [[COPY, 131072, 1, 1, 512, 8, 0, 0, 0, 5000]])
    fetch = _write(tmp_path / 'f.csv', PMC_COLS, [[COPY, 131072, 'FETCH_SIZE', 32768.0], [k, 1024, 'FETCH_SIZE', 1000.0]])
    write = _write(tmp_path / 'w.csv', PMC_COLS, [[COPY, 131072, 'WRITE_SIZE', 65536.0], [k, 1024, 'WRITE_SIZE', 500.0]])
    # MFMA busy = 8192 / (80 / 8 x 1024 SIMD-cycles) = 80%
    sq = _write(tmp_path / 's.csv', PMC_COLS, [[k, 1024, 'SQ_VALU_MFMA_BUSY_CYCLES', 8192.0],
                                               [k, 1024, 'GRBM_GUI_ACTIVE', 80.0]])
    table, sf, sw = bench.counters_from(trace, fetch, write, sq)
    assert sf == pytest.approx(2.0) and sw == pytest.approx(1.0)
    rows = [line for line in table.splitlines() if line.startswith('| `')]
    assert len(rows) == 1  # the copy is the calibration, not a row
    # 10 us; read 1000 KiB x 2 = 2.05 MB, written 500 KiB = 0.51 MB; (2048000 + 512000) B / 10 us = 256 GB/s
    assert rows[0] == '| `_ZN3kad5k_fooE` | 1024 | 3 | 10.00 | 2.05 | 0.51 | 256 | 3.2% | 80.0% |'
