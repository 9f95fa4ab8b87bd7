"""Known-answer tests of the oracle's 6502 (the NES 2A03 core: no decimal mode).

The reference's CPU core is upstream NeSLE, which is not in the reference tree, so these tests pin the oracle to
the 6502 datasheet instead, each from a formulation independent of the oracle's code:
  * cycle counts of all 151 official opcodes from the datasheet's rules per operation class and addressing mode,
    plus the page-cross and branch penalties;
  * ADC/SBC flags from signed/unsigned integer arithmetic over every (A, operand) pair;
  * compare, shift/rotate, increment, BIT and load flags from their definitions;
  * addressing quirks: zero-page index wrap, (zp,X) pointer wrap, JMP ($xxFF) page wrap, RAM mirroring;
  * stack discipline of JSR/RTS, BRK/RTI, PHP/PLP (B and unused bits), NMI entry;
  * an opcode outside the official set is a fault pc << 8 | opcode (rl/csrc/nes_machine.cuh:84-87).
"""
import numpy as np
import pytest

from helpers import Console
from rl import synth

C, Z, I, D, B, U, V, N = 1, 2, 4, 8, 16, 32, 64, 128
CODE = 0x0300


def rom_with_vectors(nmi=0xC000, reset=0xC000, irq=0xC010):
    prg = bytearray(16384)
    prg[0:3] = bytes((0x4C, 0x00, 0xC0))        # $C000: JMP $C000
    prg[0x10:0x13] = bytes((0x4C, 0x10, 0xC0))  # $C010: JMP $C010
    prg[0x3FFA:0x4000] = bytes((nmi & 0xFF, nmi >> 8, reset & 0xFF, reset >> 8, irq & 0xFF, irq >> 8))
    return synth.ines(bytes(prg), bytes(8192), 0)


@pytest.fixture
def cpu():
    return Machine()


class Machine:
    """One oracle console running code placed in RAM at $0300."""

    def __init__(self):
        self.con = Console(rom_with_vectors())

    def load(self, code, a=0, x=0, y=0, p=I | U, sp=0xFD, pc=CODE):
        ram = self.con.ram()
        ram[pc:pc + len(code)] = np.frombuffer(bytes(code), np.uint8)
        for k, v in dict(a=a, x=x, y=y, p=p, sp=sp).items():
            self.con.set(k, v)
        self.con.set('pc', pc, 'H')

    def step(self):
        cyc, fault = self.con.step()
        assert fault == 0, f'fault {fault:#x}'
        return cyc

    def reg(self, k):
        return self.con.u(k, 'H' if k == 'pc' else 'B')

    @property
    def ram(self):
        return self.con.ram()


# ---------------------------------------------------------------------------------------------- cycles

READS = {'ADC', 'AND', 'CMP', 'EOR', 'LDA', 'ORA', 'SBC', 'BIT', 'LDX', 'LDY', 'CPX', 'CPY'}
STORES = {'STA', 'STX', 'STY'}
RMW = {'ASL', 'LSR', 'ROL', 'ROR', 'INC', 'DEC'}
BRANCHES = {'BCC', 'BCS', 'BEQ', 'BMI', 'BNE', 'BPL', 'BVC', 'BVS'}


def datasheet_cycles(mn, mode):
    """Base cycles from the datasheet's rules (no page cross, branch not taken)."""
    if mn in READS:
        return dict(imm=2, zp=3, zpx=4, zpy=4, abs=4, abx=4, aby=4, izx=6, izy=5)[mode]
    if mn in STORES:
        return dict(zp=3, zpx=4, zpy=4, abs=4, abx=5, aby=5, izx=6, izy=6)[mode]
    if mn in RMW:
        return dict(acc=2, zp=5, zpx=6, abs=6, abx=7)[mode]
    if mn in BRANCHES:
        return 2
    return dict(PHA=3, PHP=3, PLA=4, PLP=4, JSR=6, RTS=6, RTI=6, BRK=7).get(mn, 3 if mn == 'JMP' and mode == 'abs'
                                                                           else 5 if mn == 'JMP' else 2)


def operands(mode):
    """Operand bytes that keep every access inside RAM without page crossing."""
    return {'imp': b'', 'acc': b'', 'imm': b'\x05', 'zp': b'\x40', 'zpx': b'\x40', 'zpy': b'\x40', 'abs': b'\x00\x04',
            'abx': b'\x00\x04', 'aby': b'\x00\x04', 'izx': b'\x20', 'izy': b'\x20', 'rel': b'\x10',
            'ind': b'\x00\x05'}[mode]


def test_all_official_opcodes_take_their_datasheet_cycles(cpu):
    assert len(synth.OPCODES) == 151
    for op, (mn, mode) in sorted(synth.OPCODES.items()):
        cpu.load(bytes([op]) + operands(mode), sp=0xF0)
        cpu.ram[0x20:0x22] = (0x00, 0x04)     # (zp) pointers -> $0400
        cpu.ram[0x500:0x502] = (0x00, 0x03)   # JMP ($0500) -> $0300
        if mn in BRANCHES:                      # make every branch not taken
            flag = {'BCC': C, 'BCS': 0, 'BEQ': 0, 'BMI': 0, 'BNE': Z, 'BPL': N, 'BVC': V, 'BVS': 0}[mn]
            cpu.con.set('p', flag | U | I)
        assert cpu.step() == datasheet_cycles(mn, mode), (hex(op), mn, mode)


@pytest.mark.parametrize('mn,op', [('LDA', 0xBD), ('LDA', 0xB9), ('EOR', 0x5D), ('LDY', 0xBC), ('LDX', 0xBE)])
def test_indexed_read_page_cross_costs_one_cycle(cpu, mn, op):
    cpu.load(bytes([op, 0xF0, 0x04]), x=0x20, y=0x20)
    assert cpu.step() == 5
    cpu.load(bytes([op, 0x00, 0x04]), x=0x20, y=0x20)
    assert cpu.step() == 4


def test_store_and_rmw_never_pay_the_page_cross(cpu):
    for op, cyc in ((0x9D, 5), (0x99, 5), (0x1E, 7), (0xFE, 7)):
        cpu.load(bytes([op, 0xF0, 0x04]), x=0x20, y=0x20)
        assert cpu.step() == cyc


def test_izy_page_cross(cpu):
    cpu.load(bytes([0xB1, 0x20]), y=0x20)
    cpu.ram[0x20:0x22] = (0xF0, 0x04)
    assert cpu.step() == 6 and cpu.reg('a') == cpu.ram[0x510]


def test_branch_cycles_and_targets(cpu):
    cpu.load(bytes([0xD0, 0x10]), p=U)             # BNE taken, same page
    assert cpu.step() == 3 and cpu.reg('pc') == CODE + 2 + 0x10
    cpu.load(bytes([0xD0, 0x80]), p=U)             # backwards across a page: $0302 - 128 = $0282
    assert cpu.step() == 4 and cpu.reg('pc') == 0x0282
    cpu.load(bytes([0xD0, 0x80]), p=U | Z)         # not taken
    assert cpu.step() == 2 and cpu.reg('pc') == CODE + 2


# ----------------------------------------------------------------------------------------- arithmetic

def signed(v):
    return v - 256 if v >= 128 else v


def test_adc_flags_exhaustive(cpu):
    for a in range(256):
        for m in range(256):
            cin = (a ^ m) & 1
            cpu.load(bytes([0x69, m]), a=a, p=U | cin)
            cpu.step()
            total = a + m + cin
            res = total & 0xFF
            s = signed(a) + signed(m) + cin
            want = (C if total > 255 else 0) | (V if not -128 <= s <= 127 else 0) | (Z if res == 0 else 0) | \
                   (N if res & 0x80 else 0)
            p = cpu.reg('p')
            assert cpu.reg('a') == res and p & (C | V | Z | N) == want, (a, m, cin)


def test_sbc_flags_exhaustive(cpu):
    for a in range(256):
        for m in range(0, 256, 3):
            cin = (a + m) & 1
            cpu.load(bytes([0xE9, m]), a=a, p=U | cin)
            cpu.step()
            diff = a - m - (1 - cin)
            res = diff & 0xFF
            s = signed(a) - signed(m) - (1 - cin)
            want = (C if diff >= 0 else 0) | (V if not -128 <= s <= 127 else 0) | (Z if res == 0 else 0) | \
                   (N if res & 0x80 else 0)
            assert cpu.reg('a') == res and cpu.reg('p') & (C | V | Z | N) == want, (a, m, cin)


def test_decimal_flag_is_ignored(cpu):
    cpu.load(bytes([0x69, 0x05]), a=0x09, p=U | D)
    cpu.step()
    assert cpu.reg('a') == 0x0E


@pytest.mark.parametrize('op,reg', [(0xC9, 'a'), (0xE0, 'x'), (0xC0, 'y')])
def test_compare_flags(cpu, op, reg):
    for r in range(0, 256, 7):
        for m in range(0, 256, 5):
            cpu.load(bytes([op, m]), **{reg: r})
            cpu.step()
            p = cpu.reg('p')
            assert bool(p & C) == (r >= m) and bool(p & Z) == (r == m) and bool(p & N) == bool((r - m) & 0x80)


def test_shifts_and_rotates(cpu):
    for v in range(256):
        for cin in (0, 1):
            for op, f in ((0x0A, lambda v, c: ((v << 1) & 0xFF, v >> 7)), (0x4A, lambda v, c: (v >> 1, v & 1)),
                          (0x2A, lambda v, c: (((v << 1) | c) & 0xFF, v >> 7)),
                          (0x6A, lambda v, c: ((v >> 1) | (c << 7), v & 1))):
                cpu.load(bytes([op]), a=v, p=U | cin)
                cpu.step()
                res, cout = f(v, cin)
                p = cpu.reg('p')
                assert cpu.reg('a') == res and (p & C) == cout and bool(p & Z) == (res == 0) and \
                    bool(p & N) == bool(res & 0x80), (hex(op), v, cin)


def test_rmw_on_memory_and_inc_dec(cpu):
    cpu.load(bytes([0xE6, 0x40]))                 # INC $40
    cpu.ram[0x40] = 0xFF
    cpu.step()
    assert cpu.ram[0x40] == 0 and cpu.reg('p') & Z
    cpu.load(bytes([0xC6, 0x41]))                 # DEC $41
    cpu.ram[0x41] = 0x00
    cpu.step()
    assert cpu.ram[0x41] == 0xFF and cpu.reg('p') & N
    cpu.load(bytes([0x7E, 0x00, 0x04]), x=3, p=U | C)   # ROR $0400,X with carry in
    cpu.ram[0x403] = 0x02
    cpu.step()
    assert cpu.ram[0x403] == 0x81 and not cpu.reg('p') & C


def test_bit(cpu):
    for m in (0x00, 0x40, 0x80, 0xC0, 0x3F):
        cpu.load(bytes([0x24, 0x40]), a=0x0F)
        cpu.ram[0x40] = m
        cpu.step()
        p = cpu.reg('p')
        assert bool(p & N) == bool(m & 0x80) and bool(p & V) == bool(m & 0x40) and bool(p & Z) == ((m & 0x0F) == 0)


def test_transfers_and_txs_flags(cpu):
    cpu.load(bytes([0xAA]), a=0x80)               # TAX sets N
    cpu.step()
    assert cpu.reg('x') == 0x80 and cpu.reg('p') & N
    cpu.load(bytes([0x9A]), x=0x00, p=U)          # TXS leaves the flags alone
    cpu.step()
    assert cpu.reg('sp') == 0 and not cpu.reg('p') & Z


# ---------------------------------------------------------------------------------------- addressing

def test_zero_page_index_wraps(cpu):
    cpu.load(bytes([0xB5, 0xFF]), x=2)            # LDA $FF,X reads $01
    cpu.ram[0x01] = 0x5A
    cpu.ram[0x101] = 0xA5
    cpu.step()
    assert cpu.reg('a') == 0x5A


def test_izx_pointer_wraps_in_zero_page(cpu):
    cpu.load(bytes([0xA1, 0xFE]), x=1)            # pointer at $FF/$00
    cpu.ram[0xFF], cpu.ram[0x00] = 0x34, 0x04
    cpu.ram[0x434] = 0x77
    cpu.step()
    assert cpu.reg('a') == 0x77


def test_jmp_indirect_page_wrap(cpu):
    cpu.load(bytes([0x6C, 0xFF, 0x04]))           # JMP ($04FF): high byte from $0400, not $0500
    cpu.ram[0x4FF], cpu.ram[0x400], cpu.ram[0x500] = 0x10, 0x03, 0x07
    assert cpu.step() == 5 and cpu.reg('pc') == 0x0310


def test_ram_is_mirrored_every_2kb(cpu):
    cpu.load(bytes([0x8D, 0x45, 0x18]), a=0x99)   # STA $1845 -> $0045
    cpu.step()
    assert cpu.ram[0x45] == 0x99
    cpu.load(bytes([0xAD, 0x45, 0x08]))           # LDA $0845
    cpu.step()
    assert cpu.reg('a') == 0x99


# ------------------------------------------------------------------------------------------ stack

def test_jsr_rts(cpu):
    cpu.load(bytes([0x20, 0x00, 0x04]), sp=0xFD)  # JSR $0400
    cpu.ram[0x400] = 0x60                         # RTS
    assert cpu.step() == 6 and cpu.reg('pc') == 0x0400 and cpu.reg('sp') == 0xFB
    assert cpu.ram[0x1FD] == 0x03 and cpu.ram[0x1FC] == 0x02   # return address - 1 = $0302
    assert cpu.step() == 6 and cpu.reg('pc') == 0x0303 and cpu.reg('sp') == 0xFD


def test_php_plp_b_and_unused_bits(cpu):
    cpu.load(bytes([0x08]), p=U | C)              # PHP pushes B and U set
    cpu.step()
    assert cpu.ram[0x1FD] == (C | B | U)
    cpu.load(bytes([0x28]), sp=0xFC, p=U)         # PLP ignores B, forces U
    cpu.ram[0x1FD] = 0xFF
    cpu.step()
    assert cpu.reg('p') == 0xFF & ~B


def test_pha_pla(cpu):
    cpu.load(bytes([0x48]), a=0x00, sp=0x00)      # push at $0100, SP wraps to $FF
    cpu.step()
    assert cpu.ram[0x100] == 0 and cpu.reg('sp') == 0xFF
    cpu.load(bytes([0x68]), sp=0xFF)              # PLA from $0100 sets Z
    cpu.step()
    assert cpu.reg('sp') == 0x00 and cpu.reg('p') & Z


def test_brk_and_rti(cpu):
    cpu.load(bytes([0x00, 0xEA]), p=U | C, sp=0xFD)   # BRK -> IRQ vector $C010
    assert cpu.step() == 7 and cpu.reg('pc') == 0xC010
    assert cpu.ram[0x1FD] == 0x03 and cpu.ram[0x1FC] == 0x02 and cpu.ram[0x1FB] == (C | B | U)
    assert cpu.reg('p') & I
    cpu.load(bytes([0x40]), sp=0xFA, p=U | I)         # RTI back to $0302 with the pushed flags minus B
    assert cpu.step() == 6 and cpu.reg('pc') == 0x0302 and cpu.reg('p') == (C | U)


def test_nmi_entry(cpu):
    cpu.load(bytes([0xEA]), p=U | C, sp=0xFD)
    cpu.con.set('nmi_pending', 1)
    cyc = cpu.step()                                 # 7 cycles of entry + the first handler instruction
    assert cyc == 7 + 3 and cpu.reg('pc') == 0xC000  # JMP $C000 at the NMI vector
    assert cpu.ram[0x1FD] == 0x03 and cpu.ram[0x1FC] == 0x00 and cpu.ram[0x1FB] == (C | U)
    assert cpu.reg('p') & I and cpu.con.u('nmi_pending') == 0


def test_unofficial_opcode_is_a_fault(cpu):
    for op in (0x02, 0x0B, 0x1A, 0x80, 0xFF):
        cpu.load(bytes([op, 0, 0]))
        cyc, fault = cpu.con.step()
        assert cyc == 0 and fault == (CODE << 8 | op)
