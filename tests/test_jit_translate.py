"""The block translation (ghostrun-lab_amd/csrc/jit.h) as text, on the CPU: where it takes a status poll's repeated
iterations at once, and that its closed form leaves the burst counter where iterating the block would."""
import ctypes
import re

import pytest

from helpers import HIP_LIB
from rl import synth
from rl.rlenv import bind_library

SKIP = re.compile(r'if \(v >= 0x([0-9A-F]+)u\) v -= \(\(v - 0x([0-9A-F]+)u\) / 0x([0-9A-F]+)u \+ 1u\) \* 0x([0-9A-F]+)u;')


def translate(rom):
    lib = bind_library(HIP_LIB)
    out = (ctypes.c_int32 * 6)()
    text = ctypes.create_string_buffer(1 << 21)
    assert lib.rlenv_jit_translate(rom, len(rom), 0, out, text, len(text)) == 0
    return text.value.decode()


def blocks(text):
    return re.findall(r'case 0x[0-9A-F]+u: JB_\d+: \{ +// \$([0-9A-F]{4}), (\d+) instructions\n(.*?)\n\}', text, re.S)


def test_status_polls_and_only_they_take_their_iterations_at_once():
    """poll_cart polls $2002 twice at boot (BIT / BPL) and three times a frame (BIT / BPL, BIT / BVS, BIT / BVC); the
    benchmark cart only at boot. Every block with the skip is a read of $2002 and a branch back to it, two
    instructions; no other block has one."""
    for rom, expect in ((synth.poll_cart(1), 5), (synth.nrom_cart(1), 2)):
        text = translate(rom)
        found = 0
        for start, n, body in blocks(text):
            if SKIP.search(body):
                found += 1
                steps = re.findall(r'JIT_STEP\(0x([0-9A-F]{2})u, 0x[0-9A-F]+u, 0x([0-9A-F]+)u\)', body)
                assert n == '2' and len(steps) == 1, body
                op, addr = int(steps[0][0], 16), int(steps[0][1], 16)
                assert op in (0x2C, 0xAD, 0xAE, 0xAC) and addr & 0xE007 == 0x2002, body
                taken = re.search(r'br_taken<kOptab\.t\[0x([0-9A-F]{2})u\]>\(h\)\) \{ v -= 0x[0-9A-F]+u; h\.pc = 0x([0-9A-F]+)u;',
                                  body)
                assert int(taken.group(1), 16) in (0x10, 0x50, 0x70) and int(taken.group(2), 16) == int(start, 16) << 3
        assert found == expect, (found, expect)


def test_bmi_poll_takes_no_iterations_at_once():
    """BIT $2002 / BMI back to itself: taken, the read saw the vblank flag set and cleared it, so the next pass falls
    through and the iterations are not alike. The poll cart's BMI variant has such a loop (besides its five other
    polls); its block must iterate one pass at a time."""
    rom = synth.poll_cart(1, bmi=True)
    at = 0xC000 + rom[16:16 + 16384].find(bytes([0x2C, 0x02, 0x20, 0x30, 0xFB]))
    text = translate(rom)
    found = {int(start, 16): body for start, n, body in blocks(text)}
    assert at in found and 'br_taken<kOptab.t[0x30u]>' in found[at], hex(at)
    assert not SKIP.search(found[at]), found[at]
    assert sum(1 for body in found.values() if SKIP.search(body)) == 5


@pytest.mark.parametrize('cross', [0, 1])
def test_skip_leaves_the_counter_where_iterating_would(cross):
    """The burst counter v holds (room - 1) << 14 | instructions run; the poll block runs while v >= its room R (the
    entry test) and takes D = (7 + cross) << 14 - 2 off it per pass (BIT 4 cycles, a taken branch 3 or 4, two
    instructions). For every v, the closed form the translation emits equals taking D off while v >= R."""
    R = ((4 << 14) - 1) + ((4 << 14) - 1)            # jit_maxtake(BIT abs) + jit_maxtake(BPL)
    D = ((4 + 3 + cross) << 14) - 2
    for v in list(range(0, 4 * R, 997)) + [R - 1, R, R + 1, R + D - 1, R + D, (0x7FFF << 14) | 0x3FFF]:
        it = v
        while it >= R:
            it -= D
        closed = v - ((v - R) // D + 1) * D if v >= R else v
        assert closed == it, v


def test_translation_compiles_with_hiprtc():
    """The benchmark cart's translation through hiprtc, as rlenv_create compiles it (hiprtc needs no GPU): the
    device headers embedded in the library must build in hiprtc's environment too, where only what they include
    themselves is declared (a host-only typedef compiled with hipcc and failed there)."""
    lib = bind_library(HIP_LIB)
    lib.rlenv_error.restype = ctypes.c_char_p
    rom = synth.nrom_cart(1)
    out = (ctypes.c_int32 * 6)()
    text = ctypes.create_string_buffer(1 << 21)
    r = lib.rlenv_jit_translate(rom, len(rom), 1, out, text, len(text))
    assert r == 0, (lib.rlenv_error() or b'').decode()[:2000]
    assert out[0] > 0 and out[3] > 0, list(out)   # blocks, code bytes


def test_ppu_register_stores_end_their_blocks():
    """An absolute store to a PPU register ($2000-$3FFF, the mirrors included) takes the generic step outside the
    part of a frame between vblank and the pre-render line, and the burst then resumes at the next instruction, so
    the translation makes that instruction a leader: such a store is the last instruction of its block. The vblank
    I/O cart stores to every register, through mirrors too; an indexed store (STA $2000,X) is not absolute and stays
    inside its block."""
    text = translate(synth.vblank_io_cart(1))
    stores, ended = 0, 0
    regs = set()
    for start, n, body in blocks(text):
        steps = re.findall(r'JIT_STEP\(0x([0-9A-F]{2})u, 0x[0-9A-F]+u, 0x([0-9A-F]+)u\)', body)
        for i, (op, base) in enumerate(steps):
            op, base = int(op, 16), int(base, 16)
            if op in (0x8D, 0x8E, 0x8C) and 0x2000 <= base < 0x4000:
                stores += 1
                regs.add(base & 7)
                assert i == len(steps) - 1, body
                tail = body[body.rfind('JIT_STEP'):]
                assert 'JIT_STEP' not in tail[8:] and ('goto JB_' in tail or 'continue;' in tail), body
                ended += 1
    assert stores == ended and stores >= 30 and regs == {0, 1, 3, 4, 5, 6, 7}, (stores, sorted(regs))
