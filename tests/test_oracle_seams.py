"""The seam cartridge (rl/synth.py seam_cart) on the oracle, one instruction at a time: its trace holds every way
code crosses an 8 KB PRG window that the interpreter's fast path treats apart - a run off a window's last byte by
instructions of 1, 2 and 3 bytes from the $8000 and the $A000 window, branches forward and back across a window
edge, heads run at $A000 and at $C000 (both PRG modes), JMP through the page-wrapping vector, code in CPU RAM - so
that the GPU parity test on the same cartridge (test_gpu_parity.py) compares those paths and not only the easy
ones."""
import numpy as np

from helpers import Console
from rl import synth

BRANCHES = {0x10, 0x30, 0x50, 0x70, 0x90, 0xB0, 0xD0, 0xF0}
FLOW = BRANCHES | {0x00, 0x20, 0x40, 0x4C, 0x60, 0x6C}


def trace(seed, steps=300_000):
    c = Console(synth.seam_cart(seed))
    rng = np.random.default_rng(seed)
    seen = dict(run=set(), fwd=set(), back=set(), heads=set(), ram=0, jmp_ind=0)
    for i in range(steps):
        if i % 5000 == 0:
            c.set('pad', int(rng.integers(256)))
        pc = c.u('pc', 'H')
        op = c.read(pc)
        _, fault = c.step()
        assert not fault, f'fault {fault} at ${pc:04X}'
        npc = c.u('pc', 'H')
        win, nwin = pc >> 13, npc >> 13
        if pc >= 0x8000 and npc >= 0x8000 and nwin != win:
            if op not in FLOW and op in synth.OPCODES:
                length = synth._LEN[synth.OPCODES[op][1]]
                if npc == pc + length:   # (else an NMI was taken)
                    seen['run'].add((win, length))
            elif op in BRANCHES:
                off = c.read(pc + 1)
                if npc == (pc + 2 + off - (256 if off >= 128 else 0)) & 0xFFFF:
                    seen['fwd' if nwin > win else 'back'].add(win)
        if npc >= 0x8000 and (npc & 0x1FFF) < 16 and pc < npc:
            seen['heads'].add(nwin)
        seen['ram'] += synth.SEAM_RAM_CODE <= pc < synth.SEAM_RAM_CODE + 32
        seen['jmp_ind'] += op == 0x6C
    return c, seen


def test_seam_cart_crosses_every_way():
    c, seen = trace(1)
    assert seen['run'] >= {(4, 1), (4, 2), (4, 3), (5, 1), (5, 2), (5, 3)}, seen['run']
    assert seen['fwd'] >= {4, 5}, seen['fwd']
    assert seen['back'] >= {5, 6}, seen['back']
    assert seen['heads'] >= {5, 6}, seen['heads']
    assert seen['ram'] > 1000 and seen['jmp_ind'] > 50, (seen['ram'], seen['jmp_ind'])
    ram = c.ram()
    assert min(ram[synth.SEAM_HEADS], ram[synth.SEAM_RAM], ram[synth.SEAM_TAILS]) > 0


def test_seam_tails_end_on_the_last_byte():
    """Each bank's tail: the 16-byte run ends exactly at the window's last byte, its last instruction 1, 2 or 3 bytes
    long by bank; the head starts with 16 NOPs."""
    rom = synth.seam_cart(0)
    prg = np.frombuffer(rom[16:16 + 128 * 1024], np.uint8)
    for b in range(15):
        page = prg[b * 8192:(b + 1) * 8192]
        assert (page[:16] == 0xEA).all() and (page[0x1FE0:0x1FF0] == 0xEA).all()
        k, last = 0x1FF0, None
        while k < 0x2000:
            last = synth._LEN[synth.OPCODES[int(page[k])][1]]
            k += last
        assert k == 0x2000 and last == b % 3 + 1, (b, k, last)
