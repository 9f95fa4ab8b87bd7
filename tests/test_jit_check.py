"""The far-jump check of compiled code objects (ghostrun-lab_amd/csrc/jit_check.h, rlenv_jit_check), on the CPU.

A branch too far for its 16-bit offset is compiled to s_getpc_b64 / s_add_u32 / s_addc_u32 / s_setpc_b64, and the
adds overwrite SCC; the compiler does not make sure that the code at the target does not read SCC first. In the
translated kernel of the benchmark's MMC3 cart this happened at the join of the page select (a read of $9Fxx went
through the $A000 window) and the pictures and RAM differed from the oracle's. The library checks every translated
code object before it uses it; these tests pin the check on code objects built here: a hand-made far jump into
s_cselect and its safe twin, the library's own kernels as built, and a translation compiled at run time; and, with
every branch expanded into a far jump (-amdgpu-s-branch-bits=5), the library's kernels and a translation, which
hold no such place with the build's flags (-enable-tail-merge=false: merged block tails were where SCC stayed live
across a jump)."""
import ctypes
import os
import struct
import subprocess
from pathlib import Path

import pytest

from helpers import HIP_LIB
from rl import synth
from rl.rlenv import bind_library

HIPCC = '/opt/rocm/bin/hipcc'

# A kernel whose inline assembly is the compiler's far-jump sequence; at its target SCC is read (the hazard) or
# written first (safe). Built here, never launched.
FAR_JUMP = r'''
#include <hip/hip_runtime.h>
extern "C" __global__ void k_far(int* p) {
    int r;
    asm volatile("s_cmp_eq_u32 %1, 0\n\t"
                 "s_getpc_b64 s[4:5]\n"
                 "0:\n\t"
                 "s_add_u32 s4, s4, (1f - 0b) & 0xffffffff\n\t"
                 "s_addc_u32 s5, s5, (1f - 0b) >> 32\n\t"
                 "s_setpc_b64 s[4:5]\n"
                 "1:\n\t"
                 TARGET
                 "s_cselect_b32 %0, 1, 2"
                 : "=s"(r) : "s"(p[0]) : "s4", "s5", "scc");
    p[1] = r;
}
'''


def check(lib, code):
    out = (ctypes.c_int32 * 2)()
    where = ctypes.create_string_buffer(512)
    assert lib.rlenv_jit_check(code, len(code), out, where, len(where)) == 0
    return out[0], out[1], where.value.decode()


def build(tmp_path, name, source):
    src = tmp_path / f'{name}.hip'
    src.write_text(source)
    co = tmp_path / f'{name}.co'
    subprocess.run([HIPCC, '-O2', '--offload-arch=gfx950', '--cuda-device-only', '--no-gpu-bundle-output',
                    str(src), '-o', str(co)], check=True, capture_output=True)
    return co.read_bytes()


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
def test_check_finds_a_far_jump_into_live_scc(tmp_path):
    lib = bind_library(HIP_LIB)
    bad = build(tmp_path, 'bad', FAR_JUMP.replace('TARGET', ''))
    good = build(tmp_path, 'good', FAR_JUMP.replace('TARGET', '"s_cmp_eq_u32 %1, 1\\n\\t"'))
    far, hazards, where = check(lib, bad)
    assert (far, hazards) == (1, 1) and 's_cselect_b32' in where, (far, hazards, where)
    assert check(lib, good)[:2] == (1, 0)
    assert check(lib, b'not a code object')[1] == -1


def bundled_code_object(so: Path) -> bytes:
    """The gfx950 code object of a HIP shared library's offload bundle."""
    data = so.read_bytes()
    i = data.find(b'__CLANG_OFFLOAD_BUNDLE__')
    assert i >= 0
    n, p = struct.unpack_from('<Q', data, i + 24)[0], i + 32
    for _ in range(n):
        off, size, tl = struct.unpack_from('<QQQ', data, p)
        triple = data[p + 24:p + 24 + tl].decode()
        p += 24 + tl
        if triple.endswith('gfx950') and size:
            return data[i + off:i + off + size]
    raise AssertionError('no gfx950 code object')


def test_library_kernels_have_no_far_jump_into_live_scc():
    """The library's kernels as built: any far jump among them lands where SCC is written first."""
    lib = bind_library(HIP_LIB)
    far, hazards, where = check(lib, bundled_code_object(HIP_LIB))
    assert hazards == 0, (far, hazards, where)


def test_translation_compiled_at_run_time_passes_the_check():
    """A banked cart's translation through hiprtc, as rlenv_create compiles it: the code object is checked before it
    is reported compiled (out[4] far jumps, out[5] hazards)."""
    lib = bind_library(HIP_LIB)
    lib.rlenv_error.restype = ctypes.c_char_p
    rom = synth.mmc3_cart(3, blocks=6, sub_blocks=4)
    out = (ctypes.c_int32 * 6)()
    assert lib.rlenv_jit_translate(rom, len(rom), 1, out, None, 0) == 0, lib.rlenv_error()
    assert out[3] > 0 and out[5] == 0, list(out)


CSRC = Path(__file__).resolve().parents[1] / 'ghostrun-lab_amd' / 'csrc'
EVERY_BRANCH_FAR = ['-mllvm', '-amdgpu-s-branch-bits=5']


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
def test_library_kernels_hold_no_far_jump_hazard_with_every_branch_far(tmp_path):
    """The library's kernels built with the Makefile's device flags and every branch expanded into a far jump: every
    far jump lands where SCC is written first (with tail merging on, 72 of about 16,000 did not)."""
    flags = subprocess.run(['make', '-s', '-C', str(CSRC), 'flags'], check=True, capture_output=True,
                           text=True).stdout.split()
    assert '-enable-tail-merge=false' in flags
    flags = [f for f in flags if f not in ('-fPIC', '-shared')]
    co = tmp_path / 'lib.co'
    subprocess.run([HIPCC, *flags, *EVERY_BRANCH_FAR, '-I', str(CSRC / '_build'), '--cuda-device-only',
                    '--no-gpu-bundle-output', '-c', str(CSRC / 'rlenv_hip.hip'), '-o', str(co)],
                   check=True, capture_output=True, cwd=str(CSRC))
    far, hazards, where = check(bind_library(HIP_LIB), co.read_bytes())
    assert far > 10000 and hazards == 0, (far, hazards, where)


def test_translation_holds_no_far_jump_hazard_with_every_branch_far():
    """A banked cart's translation compiled with every branch expanded into a far jump (RLENV_JIT_EXTRA): the check
    passes (out[5] = 0 hazards among out[4] far jumps)."""
    lib = bind_library(HIP_LIB)
    lib.rlenv_error.restype = ctypes.c_char_p
    rom = synth.mmc3_cart(3, blocks=6, sub_blocks=4)
    out = (ctypes.c_int32 * 6)()
    os.environ['RLENV_JIT_EXTRA'] = ' '.join(EVERY_BRANCH_FAR)
    try:
        rc = lib.rlenv_jit_translate(rom, len(rom), 1, out, None, 0)
    finally:
        del os.environ['RLENV_JIT_EXTRA']
    assert rc == 0, lib.rlenv_error()
    assert out[4] > 1000 and out[5] == 0, list(out)
