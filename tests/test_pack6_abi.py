"""The lossless 6-bit frame codec on the oracle, and the C ABI of both libraries (no GPU needed).

pack6 is pinned by a bit-level formulation independent of the packing arithmetic: bit 6k+b of each little-endian
24-bit group is bit b of pixel k (rl/csrc/rlenv.cu:127-142; the reference's KAT rl/tests/test_host_obs_pack6.py:17-31
checks all 64 colours and 131,072 random quads the same way, plus the round trip).
"""
import ctypes
import re
import subprocess

import numpy as np

from helpers import HIP_LIB, ORACLE_LIB, ROOT, oracle, ptr

HEADER = ROOT / 'include' / 'rlenv_api.h'


def pack(px):
    out = np.zeros(len(px) // 4 * 3, np.uint8)
    assert oracle().rl_pack6(ptr(px), ptr(out), len(px), None) == 0
    return out


def unpack(packed, n):
    out = np.zeros(n, np.uint8)
    assert oracle().rl_unpack6(ptr(packed), ptr(out), n, None) == 0
    return out


def bits_form(px):
    """Packed bytes from the bit layout alone."""
    bits = np.unpackbits(px[:, None], axis=1, bitorder='little')[:, :6]       # [n, 6] bits of each pixel
    return np.packbits(bits.reshape(-1, 24), axis=1, bitorder='little').reshape(-1)


def test_all_colours_and_random_quads():
    rng = np.random.default_rng(0)
    px = np.concatenate([np.repeat(np.arange(64, dtype=np.uint8), 4),
                         rng.integers(0, 64, 131072 * 4, dtype=np.uint8)])
    packed = pack(px)
    assert len(packed) * 4 == len(px) * 3
    assert np.array_equal(packed, bits_form(px))
    assert np.array_equal(unpack(packed, len(px)), px)


def test_unpack_masks_six_bits_and_frame_round_trip():
    rng = np.random.default_rng(1)
    frame = rng.integers(0, 64, (4, 224, 240), dtype=np.uint8).reshape(-1)
    assert np.array_equal(unpack(pack(frame), frame.size), frame)
    packed = rng.integers(0, 256, 3 * 1000, dtype=np.uint8)
    out = unpack(packed, 4000)
    assert out.max() < 64 and np.array_equal(pack(out), packed)


def test_pixel_count_must_divide_by_four():
    px = np.zeros(6, np.uint8)
    out = np.zeros(8, np.uint8)
    lib = oracle()
    assert lib.rl_pack6(ptr(px), ptr(out), 6, None) != 0
    lib.rlenv_error.restype = ctypes.c_char_p
    assert b'four' in lib.rlenv_error()


def declared():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(rlenv_\w+|rl_\w+|rl10_\w+)\s*\(', text)))


def exported(lib):
    out = subprocess.run(['nm', '-D', '--defined-only', str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if ' T ' in line}


def test_hip_library_exports_every_declared_entry_point():
    names = declared()
    assert len(names) >= 30 and 'rlenv_step' in names and 'rl_pack6' in names
    missing = [n for n in names if n not in exported(HIP_LIB)]
    assert not missing, missing


def test_hip_library_loads_without_a_gpu():
    lib = ctypes.CDLL(str(HIP_LIB))
    for n in declared():
        assert hasattr(lib, n), n


def test_oracle_exports_the_env_abi():
    have = exported(ORACLE_LIB)
    core = [n for n in declared() if n not in ('rl_host_alloc', 'rl_host_free', 'rl_memcpy_async', 'rl_gather_rows',
                                               'rl_gather_envs', 'rl_stream_create', 'rl_stream_destroy',
                                               'rlenv_step_game', 'rlenv_step_range',
                                               'rlenv_step_static', 'rlenv_jit_translate',
                                               'rlenv_jit_check')]
    missing = [n for n in core if n not in have]
    assert not missing, missing
