"""The device build keeps packed FP32 math out of the HIP code: `-Xclang -target-feature -Xclang -packed-fp32-ops`
reaches the gfx950 device pass (hipcc's host pass is the one that warns it does not know the feature). A probe kernel
with two adjacent float multiply-adds gets a packed instruction without the flag and none with it, and the
product's device code, built with the Makefile's flags, holds no v_pk_fma_f32 / v_pk_mul_f32 / v_pk_add_f32 and no
kernel spills to scratch."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / 'ghostrun-lab_amd' / 'csrc'
HIPCC = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
NO_PACKED = ['-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops']
PACKED = re.compile(r'\bv_pk_(fma|mul|add)_f32\b')
PROBE = r'''#include <hip/hip_runtime.h>
__global__ void probe(float* a) {
    const int i = 2 * threadIdx.x;
    a[i] = a[i] * 3.0f + 1.0f;
    a[i + 1] = a[i + 1] * 3.0f + 1.0f;
}
'''

def device_asm(src, out, extra, remarks=None):
    cmd = [HIPCC, '-O3', '-std=c++17', '--offload-arch=gfx950', '--cuda-device-only', '-S', str(src), '-o', str(out),
           *extra]
    if remarks is not None:
        cmd.append('-Rpass-analysis=kernel-resource-usage')
    r = subprocess.run(cmd, check=True, capture_output=True, text=True)
    if remarks is not None:
        remarks.append(r.stderr)
    return out.read_text()


def makefile_flags():
    text = (CSRC / 'Makefile').read_text().replace('\\\n', ' ')
    flags = re.search(r'^HIPFLAGS\s*[:?]?=(.*)$', text, re.M).group(1).split()
    return [f for f in flags if f not in ('-fPIC', '-shared') and not f.startswith('-I')]


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
def test_flag_reaches_the_device_pass(tmp_path):
    src = tmp_path / 'probe.hip'
    src.write_text(PROBE)
    assert PACKED.search(device_asm(src, tmp_path / 'a.s', []))
    assert not PACKED.search(device_asm(src, tmp_path / 'b.s', NO_PACKED))


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
def test_product_device_code_has_no_packed_fp32_and_no_scratch(tmp_path):
    """Also: no kernel of the library uses scratch (private memory) - every local stays in registers or LDS."""
    flags = makefile_flags()
    assert all(f in flags for f in NO_PACKED)
    remarks = []
    asm = device_asm(CSRC / 'rlenv_hip.hip', tmp_path / 'rlenv.s', [f'-I{ROOT / "include"}', f'-I{CSRC}',
                                                                     f'-I{CSRC / "_build"}'] +
                     [f for f in flags if not f.startswith('--offload-arch') and f != '-O3' and f != '-std=c++17'],
                     remarks)
    assert '.amdgcn_target "amdgcn-amd-amdhsa--gfx950"' in asm
    assert not PACKED.search(asm)
    names = re.findall(r'Function Name: (\S+)', remarks[0])
    scratch = [int(x) for x in re.findall(r'ScratchSize \[bytes/lane\]: (\d+)', remarks[0])]
    assert len(names) == len(scratch) >= 15 and any('k_emu_w' in n for n in names)
    assert not [n for n, b in zip(names, scratch) if b], list(zip(names, scratch))


TRANSLATED = {   # cart, board class, with the frame-bank kernel (a one-game env of one round of waves)
    'nrom': (lambda synth: synth.nrom_cart(1), 'NES_BOARD_NROM', True),
    'poll-bmi': (lambda synth: synth.poll_cart(1, bmi=True), 'NES_BOARD_NROM', False),
    'mmc3': (lambda synth: synth.mmc3_cart(3, blocks=6, sub_blocks=4), 'NES_BOARD_MMC3', False),
}


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
@pytest.mark.parametrize('case', sorted(TRANSLATED))
def test_translated_kernel_device_code_has_no_packed_fp32_and_no_scratch(tmp_path, case):
    """The kernels the library compiles at run time from a cartridge's translated blocks (jit.h: frames drawn from
    frame banks, and frames the emulator's waves draw themselves, with the decision's finish), built with the same
    flags: the benchmark cart's (both kernels), the poll cart with its BMI poll, and a banked MMC3 cart's (blocks by
    PRG offset, the banked board class): no packed FP32, no scratch, 8 waves per SIMD."""
    import ctypes
    from rl import synth
    from rl.rlenv import bind_library
    from helpers import HIP_LIB
    make, board, bank = TRANSLATED[case]
    lib = bind_library(HIP_LIB)
    rom = make(synth)
    out = (ctypes.c_int32 * 6)()
    text = ctypes.create_string_buffer(1 << 21)
    assert lib.rlenv_jit_translate(rom, len(rom), 0, out, text, len(text)) == 0
    assert out[0] > 20 and out[1] > 50 and len(text.value) < len(text) - 1
    (tmp_path / 'jit_blocks.inc').write_bytes(text.value)
    src = tmp_path / 'jit.hip'
    kernels = (['k_emu_jit'] if bank else []) + ['k_emu_jit_draw']
    body = '#define RLENV_JIT_INC "jit_blocks.inc"\n#include "emu_kernel.h"\n'
    if bank:
        body += ('extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n'
                 f'void k_emu_jit(nd::EmuArgs a) {{ nd::emu_body<{board}, true, false>(a); }}\n')
    body += ('extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n'
             f'void k_emu_jit_draw(nd::EmuArgs a) {{ nd::emu_body<{board}, false, true>(a); }}\n')
    src.write_text(body)
    flags = makefile_flags()
    remarks = []
    asm = device_asm(src, tmp_path / 'jit.s', [f'-I{ROOT / "include"}', f'-I{CSRC}', f'-I{tmp_path}'] +
                     [f for f in flags if not f.startswith('--offload-arch') and f != '-O3' and f != '-std=c++17'],
                     remarks)
    assert all(k in asm for k in kernels) and not PACKED.search(asm)
    scratch = [int(x) for x in re.findall(r'ScratchSize \[bytes/lane\]: (\d+)', remarks[0])]
    occupancy = [int(x) for x in re.findall(r'Occupancy \[waves/SIMD\]: (\d+)', remarks[0])]
    assert scratch == [0] * len(kernels) and occupancy == [8] * len(kernels), (scratch, occupancy)
