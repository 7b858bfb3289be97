"""include/spmm_amd.h is C: it compiles as strict C99, and the layout a C
compiler gives its structs (the size and every field's offset) is the one the
ctypes mirrors in test_gpu_abi.py pass through the C ABI."""

import ctypes as C
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / 'include'
GCC = shutil.which('gcc')

pytestmark = pytest.mark.skipif(GCC is None, reason='no C compiler')


def test_header_compiles_as_c99():
    r = subprocess.run([GCC, '-std=c99', '-Wall', '-Wextra', '-Werror', '-pedantic', '-fsyntax-only', '-x', 'c',
                        str(INCLUDE / 'spmm_amd.h')], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_struct_layouts_match_the_ctypes_mirrors(tmp_path):
    from test_gpu_abi import BooDesc, BooHost, PbrDesc, StageInfo
    structs = {'spmm_boo_host': BooHost, 'spmm_boo_stage_info': StageInfo, 'spmm_boo_desc': BooDesc,
               'spmm_pbr_desc': PbrDesc}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "spmm_amd.h"', 'int main(void) {']
    for cname, mirror in structs.items():
        lines.append(f'    printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in mirror._fields_:
            lines.append(f'    printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ['    return 0;', '}', '']
    src, exe = tmp_path / 'layout.c', tmp_path / 'layout'
    src.write_text('\n'.join(lines))
    r = subprocess.run([GCC, '-std=c99', '-Wall', '-Werror', f'-I{INCLUDE}', str(src), '-o', str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr  # a field the mirror names but the header lacks fails here
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        name, field, value = line.split()
        got[(name, field)] = int(value)
    for cname, mirror in structs.items():
        assert got[(cname, 'sizeof')] == C.sizeof(mirror), cname
        for field, _ in mirror._fields_:
            assert got[(cname, field)] == getattr(mirror, field).offset, (cname, field)
