"""Builds libkadconv_hip.so (gfx950) in-tree from csrc/.

    python kad-conv_amd/build.py            # incremental
    python kad-conv_amd/build.py --force    # rebuild everything

Objects go to kad-conv_amd/_build/, the shared library to
kad-conv_amd/kadconv/libkadconv_hip.so, where kadconv._ext loads it.
"""
import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
OBJ = os.path.join(HERE, '_build')
LIB = os.path.join(HERE, 'kadconv', 'libkadconv_hip.so')
INCLUDE = os.path.join(os.path.dirname(HERE), 'include')
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
ARCH = 'gfx950'
# Packed FP32 VALU ops are disabled for all device code (see the kernels' notes).
FLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}', '-I', CSRC, '-I', INCLUDE,
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', '-Wno-unused-result']


def _deps():
    return glob.glob(os.path.join(CSRC, '*.h')) + [os.path.join(INCLUDE, 'kadconv_hip.h')]


def _compile(src, force):
    obj = os.path.join(OBJ, os.path.basename(src) + '.o')
    newest = max([os.path.getmtime(src)] + [os.path.getmtime(d) for d in _deps()])
    if not force and os.path.exists(obj) and os.path.getmtime(obj) >= newest:
        return obj, None
    cmd = [HIPCC] + FLAGS + ['-c', src, '-o', obj]
    if src.endswith('.cpp'):
        cmd[1:1] = ['-x', 'hip']
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        return obj, f'{" ".join(cmd)}\n{r.stdout}\n{r.stderr}'
    return obj, None


def build(force=False, jobs=8, verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, '*.hip')) + glob.glob(os.path.join(CSRC, '*.cpp')))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda s: _compile(s, force), srcs))
    errs = [e for _, e in results if e]
    if errs:
        raise RuntimeError('HIP build failed:\n' + '\n'.join(errs))
    objs = [o for o, _ in results]
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < max(os.path.getmtime(o) for o in objs):
        tmp = LIB + '.tmp'
        cmd = [HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', tmp] + objs
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f'link failed:\n{" ".join(cmd)}\n{r.stdout}\n{r.stderr}')
        os.replace(tmp, LIB)
    if verbose:
        print('built', LIB)
    return LIB


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('--force', action='store_true')
    ap.add_argument('-j', type=int, default=8)
    args = ap.parse_args()
    build(force=args.force, jobs=args.j, verbose=True)
    sys.exit(0)
