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


@pytest.mark.skipif(not Path(HIPCC).exists(), reason='hipcc not installed')
def test_translated_kernel_device_code_has_no_packed_fp32_and_no_scratch(tmp_path):
    """The kernels the library compiles at run time from a cartridge's translated blocks (jit.h: frames drawn from
    frame banks, and frames the emulator's waves draw themselves, with the decision's finish), here the blocks of the
    benchmark cart (rl.synth.nrom_cart(1)) as rlenv_jit_translate writes them, built with the same flags."""
    import ctypes
    from rl import synth
    from rl.rlenv import bind_library
    from helpers import HIP_LIB
    lib = bind_library(HIP_LIB)
    rom = synth.nrom_cart(1)
    out = (ctypes.c_int32 * 6)()
    text = ctypes.create_string_buffer(1 << 20)
    assert lib.rlenv_jit_translate(rom, len(rom), 0, out, text, len(text)) == 0
    assert out[0] > 50 and out[1] > 200 and len(text.value) < len(text) - 1
    (tmp_path / 'jit_blocks.inc').write_bytes(text.value)
    src = tmp_path / 'jit.hip'
    src.write_text('#define RLENV_JIT_INC "jit_blocks.inc"\n#include "emu_kernel.h"\n'
                   'extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n'
                   'void k_emu_jit(nd::EmuArgs a) { nd::emu_body<NES_BOARD_NROM, true, false>(a); }\n'
                   'extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n'
                   'void k_emu_jit_draw(nd::EmuArgs a) { nd::emu_body<NES_BOARD_NROM, false, true>(a); }\n')
    flags = makefile_flags()
    remarks = []
    asm = device_asm(src, tmp_path / 'jit.s', [f'-I{ROOT / "include"}', f'-I{CSRC}', f'-I{tmp_path}'] +
                     [f for f in flags if not f.startswith('--offload-arch') and f != '-O3' and f != '-std=c++17'],
                     remarks)
    assert 'k_emu_jit' in asm and 'k_emu_jit_draw' in asm and not PACKED.search(asm)
    scratch = [int(x) for x in re.findall(r'ScratchSize \[bytes/lane\]: (\d+)', remarks[0])]
    occupancy = [int(x) for x in re.findall(r'Occupancy \[waves/SIMD\]: (\d+)', remarks[0])]
    assert scratch == [0, 0] and occupancy == [8, 8], (scratch, occupancy)
