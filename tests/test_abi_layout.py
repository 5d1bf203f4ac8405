"""The ctypes mirrors of the argument structs in kadconv/_ext.py have the layout that
include/kadconv_hip.h gives them: a C program built with gcc from the header prints
sizeof and every field's offsetof, compared with ctypes' (no GPU needed)."""
import ctypes
import os
import shutil
import subprocess

import pytest

from tests.conftest import ROOT

STRUCTS = {'kad_dcn_args': 'DcnArgs', 'kad_lcsa_args': 'LcsaArgs', 'kad_gemm_args': 'GemmArgs',
           'kad_pyramid_args': 'PyramidArgs', 'kad_merge_args': 'MergeArgs', 'kad_resample_args': 'ResampleArgs',
           'kad_decode_args': 'DecodeArgs'}


@pytest.mark.skipif(shutil.which('gcc') is None, reason='needs gcc')
def test_ctypes_structs_match_header(tmp_path):
    from kadconv import _ext
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "kadconv_hip.h"', 'int main(void) {']
    expect = []
    for cname, pyname in STRUCTS.items():
        cls = getattr(_ext, pyname)
        lines.append(f'  printf("%zu\\n", sizeof({cname}));')
        expect.append(ctypes.sizeof(cls))
        for field in cls._fields_:
            lines.append(f'  printf("%zu\\n", offsetof({cname}, {field[0]}));')
            expect.append(getattr(cls, field[0]).offset)
    lines += ['  return 0;', '}']
    src = tmp_path / 'layout.c'
    src.write_text('\n'.join(lines) + '\n')
    exe = tmp_path / 'layout'
    subprocess.run(['gcc', '-std=c11', '-I', os.path.join(ROOT, 'include'), str(src), '-o', str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got == expect
