"""In-tree build of the native parts of spmm_amd.

Two artefacts, both next to this file:

* ``libspmm_amd.so`` -- the HIP kernels and the C ABI of ``include/spmm_amd.h``,
  compiled by hipcc for gfx950 only;
* ``_core.<abi>.so`` -- the pybind11 host layer (format builders, CPU ops, GPU
  glue), compiled by g++ and linked against ``libspmm_amd.so`` through an
  ``$ORIGIN`` rpath.

``python spmm_amd/build.py`` rebuilds both (run by path: importing the package
needs the libraries this script builds).  Nothing is JIT-compiled at import
time: ``spmm_amd`` loads what is here and fails loudly when it is missing.

Host-code sanitizers (CPU only; the GPU code is never built with them):

* ``python spmm_amd/build.py core-san`` -- ``_core`` with AddressSanitizer and
  UBSan (every UB check fatal) into ``_build/san/``, linked against a copy of
  the C ABI library whose host code (the tile-stream staging among it) is
  built with the same checks (``libspmm_amd_san.so``);
* ``python spmm_amd/build.py san-test [pytest args]`` -- builds it and runs
  ``pytest -m "not gpu"`` with that module loaded in place of ``_core``
  (``SPMM_AMD_CORE``), the tests that open the C ABI with ctypes on that
  library (``SPMM_AMD_LIB``), and the sanitizer runtimes preloaded into Python.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / 'csrc'
INCLUDE = ROOT / 'include'

HIP_LIB = HERE / 'libspmm_amd.so'
CORE_LIB = HERE / ('_core' + sysconfig.get_config_var('EXT_SUFFIX'))

ARCH = os.environ.get('SPMM_AMD_ARCH', 'gfx950')

# Packed-FP32 instructions are disabled for all device code: hipcc -O3 would
# otherwise form v_pk_{add,mul,fma}_f32 from plain float code.
HIPCC_FLAGS = [
    '-O3', '-std=c++17', f'--offload-arch={ARCH}', '-fPIC', '-shared',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-function', '-pthread',
]

# -ffp-contract=off keeps the CPU ops' y += a*x as a separate multiply and add,
# the rounding of the reference's CPU loops.
CXX_FLAGS = ['-O3', '-std=c++17', '-fPIC', '-shared', '-ffp-contract=off', '-fvisibility=hidden', '-pthread']


def _run(cmd):
    print('+', ' '.join(str(c) for c in cmd), flush=True)
    subprocess.run([str(c) for c in cmd], check=True)


def _hipcc():
    for cand in (os.environ.get('HIPCC'), '/opt/rocm/bin/hipcc', 'hipcc'):
        if cand and (os.path.sep not in cand or Path(cand).exists()):
            return cand
    return 'hipcc'


def build_hip(out=HIP_LIB, extra=()):
    srcs = [CSRC / 'spmm_kernels.hip', CSRC / 'measure.hip']
    # measure.hip opens librocsparse with dlopen: link libdl only
    _run([_hipcc(), *HIPCC_FLAGS, *extra, f'-I{INCLUDE}', *srcs, '-o', out, '-ldl'])


def build_core(out=CORE_LIB, flags=CXX_FLAGS, rpath='$ORIGIN', lib='spmm_amd', libdir=HERE):
    import pybind11
    src = CSRC / 'core.cpp'
    py_inc = sysconfig.get_paths()['include']
    _run(['g++', *flags, f'-I{INCLUDE}', f'-I{CSRC}', f'-I{pybind11.get_include()}',
          f'-I{py_inc}', src, '-o', out, f'-L{libdir}', f'-l{lib}', f'-Wl,-rpath,{rpath}'])


SAN_DIR = ROOT / '_build' / 'san'
SAN_CORE = SAN_DIR / CORE_LIB.name
SAN_FLAGS = ['-O1', '-g', '-fno-omit-frame-pointer', '-fsanitize=address,undefined',
             '-fno-sanitize-recover=all', *[f for f in CXX_FLAGS if f != '-O3']]
# The C ABI library again with its host code -- the tile-stream staging, the
# entry points' checks -- under the same sanitizers; each flag is passed to
# the host compilation only (-Xarch_host), the GPU code is built as usual.
SAN_LIB = SAN_DIR / 'libspmm_amd_san.so'
# The runtimes preloaded are gcc's (the core is built by g++); clang's
# function-type check is the one UBSan check they have no handler for.
SAN_HOST_FLAGS = ['-Xarch_host', '-g', '-Xarch_host', '-fno-omit-frame-pointer',
                  '-Xarch_host', '-fsanitize=address',
                  '-Xarch_host', '-fsanitize=undefined',
                  '-Xarch_host', '-fno-sanitize=function',
                  '-Xarch_host', '-fno-sanitize-recover=all',
                  f'-Wl,-soname,{SAN_LIB.name}']


def build_core_san():
    SAN_DIR.mkdir(parents=True, exist_ok=True)
    build_hip(SAN_LIB, SAN_HOST_FLAGS)
    build_core(SAN_CORE, SAN_FLAGS, str(SAN_DIR), lib='spmm_amd_san', libdir=SAN_DIR)


def san_env():
    runtimes = []
    for lib in ('libasan.so', 'libubsan.so'):
        path = subprocess.run(['g++', f'-print-file-name={lib}'], check=True, capture_output=True,
                              text=True).stdout.strip()
        runtimes.append(path)
    env = dict(os.environ)
    env.update(SPMM_AMD_CORE=str(SAN_CORE), SPMM_AMD_LIB=str(SAN_LIB), LD_PRELOAD=' '.join(runtimes),
               # Python and torch are not instrumented: their allocations are
               # outside the checks, and their exit-time leaks are not ours
               ASAN_OPTIONS='detect_leaks=0:alloc_dealloc_mismatch=0:abort_on_error=1',
               UBSAN_OPTIONS='print_stacktrace=1:halt_on_error=1')
    return env


def san_test(args):
    build_core_san()
    cmd = [sys.executable, '-m', 'pytest', str(ROOT / 'tests'), '-q', '-m', 'not gpu', '-p',
           'no:cacheprovider', *args]
    print('+', ' '.join(cmd), flush=True)
    sys.exit(subprocess.run(cmd, env=san_env(), cwd=ROOT).returncode)


def build_all():
    build_hip()
    build_core()


if __name__ == '__main__':
    which = sys.argv[1:] or ['all']
    if which[0] == 'san-test':
        san_test(which[1:])
    for w in which:
        {'all': build_all, 'hip': build_hip, 'core': build_core, 'core-san': build_core_san}[w]()
