"""Known-answer tests of the oracle's cartridge boards (NROM, UxROM, CNROM, MMC1, MMC3, MMC2) and its DMC.

MMC3: restates the reference's register case third_party/nesle-extensions.patch:4638-4673 (R0-R7 = 00 3A 4A 5D 6E 61
0A 04, bank select $46, $A000 = 1 on 128 KB PRG / 128 KB CHR) by writing the registers through the CPU bus, plus
the scanline counter (reload, count down once per rendered line at dot 266, IRQ at zero, $E000 acknowledge).
MMC1: the serial port and the bank modes written from the board's documented register meanings (16 KB PRG banks,
4 KB CHR banks), not from the oracle's page arithmetic.
UxROM / CNROM: the bank latch and its declared AND-type bus conflicts from the board's behaviour as the reference states it
(patch:2982-2990, 3124-3127, 4008), checked on a cart whose PRG pages are tagged with their numbers.
MMC2: the registers, the CPU-driven latch flips and the renderer's fetch-then-flip order along a line as the reference
states them (patch:3027-3035, 3147-3156, 3196-3220, 1385-1402, 1548-1551).
DMC: restates the sample-channel cases of patch:4105-4205 (status bit 4, 4-cycle fetch steals, loop, rate change,
no steal in the idle fast-forward) with the same 4-cycle instruction driver as the reference test.
"""
import numpy as np
import pytest

from helpers import Console, ptr
from rl import synth

KB = 1024


def cart(mapper, prg_kb, chr_kb, vertical=True):
    prg = bytearray(prg_kb * KB)
    for i in range(0, len(prg), 8 * KB):                 # tag every 8 KB page with its number
        prg[i] = i // (8 * KB)
    last = len(prg) - 8 * KB
    prg[last + 0x10:last + 0x14] = bytes((0xEA, 0x4C, 0x10, 0xE0))  # $E010: NOP; JMP $E010
    prg[-6:] = bytes((0x10, 0xE0, 0x10, 0xE0, 0x10, 0xE0))
    return synth.ines(bytes(prg), bytes(chr_kb * KB), mapper, vertical=vertical)


def pages(con):
    return ([int(x) // (8 * KB) for x in con.words('prg_off', 4)], [int(x) // KB for x in con.words('chr_off', 8)],
            [int(x) for x in con.mem('nt_map', 4)])


# ----------------------------------------------------------------------------------------------- NROM

def test_nrom_128_is_mirrored_and_header_mirroring():
    con = Console(cart(0, 16, 8, vertical=False))
    prg, chr_, nt = pages(con)
    assert [con.read(a) for a in (0x8000, 0xA000, 0xC000, 0xE000)] == [0, 1, 0, 1]
    assert chr_ == list(range(8)) and nt == [0, 0, 1, 1]
    assert pages(Console(cart(0, 32, 8)))[2] == [0, 1, 0, 1]


# ---------------------------------------------------------------------------------------------- CNROM

def cnrom_cart(conflicts):
    """32 KB PRG (8 KB pages tagged with their number), 32 KB CHR; NES 2.0 submapper 2 when conflicts."""
    prg = bytearray(32 * KB)
    for i in range(0, len(prg), 8 * KB):
        prg[i] = i // (8 * KB)
    prg[0x7FF0] = 0x0C                                   # a ROM byte with bits 2-3 set
    prg[0x6010:0x6014] = bytes((0xEA, 0x4C, 0x10, 0xE0))
    prg[-6:] = bytes((0x10, 0xE0, 0x10, 0xE0, 0x10, 0xE0))
    return synth.ines(bytes(prg), bytes(32 * KB), 3, submapper=2 if conflicts else None)


def test_cnrom_bank_latch():
    """The 8 KB CHR bank is the written value, masked to the CHR size; PRG stays fixed (patch:2982-2990,
    3124-3127)."""
    con = Console(cnrom_cart(False))
    prg, chr_, nt = pages(con)
    assert chr_ == list(range(8)) and [con.read(a) for a in (0x8000, 0xA000, 0xC000, 0xE000)] == [0, 1, 2, 3]
    con.write(0x8000, 2)
    assert pages(con)[1] == list(range(16, 24))
    con.write(0xFFF0, 7)                                 # 4 banks: 7 -> 3
    assert pages(con)[1] == list(range(24, 32))
    assert [con.read(a) for a in (0x8000, 0xA000, 0xC000, 0xE000)] == [0, 1, 2, 3]


def test_cnrom_declared_bus_conflicts():
    """Declared AND-type bus conflicts (NES 2.0 submapper 2): the latch takes value AND the ROM byte under the
    address; the same writes on an iNES 1.0 header take the value (patch:4008)."""
    con = Console(cnrom_cart(True))
    con.write(0xA000, 3)                                 # ROM byte 1
    assert pages(con)[1] == list(range(8, 16))
    con.write(0xFFF0, 0xFF)                              # ROM byte $0C -> 0x0C & 3 = 0 after the mask
    assert pages(con)[1] == list(range(8))
    con.write(0xC000, 0x07)                              # ROM byte 2
    assert pages(con)[1] == list(range(16, 24))
    plain = Console(cnrom_cart(False))
    plain.write(0xA000, 3)
    assert pages(plain)[1] == list(range(24, 32))


@pytest.mark.parametrize('conflicts', [False, True])
def test_cnrom_synthetic_cart_switches_chr(conflicts):
    """The seed-generated CNROM cart (the GPU parity case) selects all four CHR banks, some of them mid-frame
    (frame-log CHR events), with and without declared bus conflicts."""
    con = Console(synth.cnrom_cart(1, conflicts=conflicts))
    t, banks, events = 82182, set(), 0
    for f in range(40):
        con.set('pad', [0x81, 0x40, 0x02, 0xC0][f % 4])
        assert con.run_until(t) == 0
        t += 89342
        banks.add(pages(con)[1][0] // 8)
        n = con.u('log_n', 'H')
        log = con.words('log', 16 + 2 * 256)
        events += sum(1 for i in range(min(n, 256)) if (int(log[16 + 2 * i]) & 15) == 7)   # NES_EV_CHR
    assert banks == {0, 1, 2, 3} and events > 0


# ---------------------------------------------------------------------------------------------- UxROM

def test_uxrom_bank_at_8000_last_bank_fixed():
    """The 16 KB bank at $8000 is the written value, masked to the PRG size; the last 16 KB stay at $C000."""
    con = Console(cart(2, 128, 8))
    assert [con.read(a) for a in (0x8000, 0xA000, 0xC000, 0xE000)] == [0, 1, 14, 15]
    con.write(0xC000, 3)                                 # no conflicts declared: ROM byte 14 does not matter
    assert [con.read(a) for a in (0x8000, 0xA000, 0xC000, 0xE000)] == [6, 7, 14, 15]
    con.write(0x8001, 0x0B)                              # 8 banks: 11 -> 3
    assert pages(con)[0] == [6, 7, 14, 15] and pages(con)[1] == list(range(8))


def test_uxrom_declared_bus_conflicts():
    """Declared AND-type bus conflicts: the bank is value AND the ROM byte under the address."""
    prg = bytearray(128 * KB)
    for i in range(0, len(prg), 8 * KB):
        prg[i] = i // (8 * KB)
    prg[-6:] = bytes((0x10, 0xE0, 0x10, 0xE0, 0x10, 0xE0))
    con = Console(synth.ines(bytes(prg), bytes(8 * KB), 2, submapper=2))
    con.write(0xC000, 0x07)                              # ROM byte 14: 7 & 14 = 6
    assert pages(con)[0] == [12, 13, 14, 15]
    con.write(0xA000, 0x07)                              # ROM byte at $A000 = tag of page 13: 7 & 13 = 5
    assert pages(con)[0] == [10, 11, 14, 15]


@pytest.mark.parametrize('conflicts', [False, True])
def test_uxrom_synthetic_cart_switches_banks(conflicts):
    """The seed-generated UxROM cart (the GPU parity case) selects the switchable banks and calls into them."""
    con = Console(synth.uxrom_cart(1, conflicts=conflicts))
    t, seen = 82182, set()
    for f in range(40):
        con.set('pad', [0x81, 0x40, 0x02, 0xC0][f % 4])
        assert con.run_until(t) == 0
        t += 89342
        seen.add(pages(con)[0][0] // 2)
    assert len(seen) >= 4


# ----------------------------------------------------------------------------------------------- MMC3

def mmc3_write_regs(con, regs, select, mirror):
    for r, v in enumerate(regs):
        con.write(0x8000, r)
        con.write(0x8001, v)
    con.write(0x8000, select)
    con.write(0xA000, mirror)


def test_mmc3_register_case_of_the_reference():
    con = Console(cart(4, 128, 128))
    mmc3_write_regs(con, (0, 0x3A, 0x4A, 0x5D, 0x6E, 0x61, 0x0A, 0x04), 0x46, 1)
    prg, chr_, nt = pages(con)
    # PRG mode 1: R6 at $C000, the second-last page at $8000, R7 at $A000, the last page fixed at $E000
    assert prg == [0x7E & 15, 0x04, 0x0A, 15]
    assert [con.read(a) for a in (0x8000, 0xA000, 0xC000)] == [14, 4, 10]
    # no CHR inversion: R0/R1 as 2 KB banks at $0000/$0800, R2-R5 as 1 KB banks at $1000-$1C00
    assert chr_[2:4] == [0x3A, 0x3B] and chr_[4] == 0x4A and chr_[7] == 0x61 and chr_[0:2] == [0, 1]
    assert nt == [0, 0, 1, 1]                            # $A000 bit 0 = 1: horizontal


def test_mmc3_chr_inversion_and_prg_mode0():
    con = Console(cart(4, 256, 128))
    mmc3_write_regs(con, (0x10, 0x21, 0x30, 0x31, 0x32, 0x33, 0x05, 0x06), 0x80, 0)
    prg, chr_, nt = pages(con)
    assert prg == [5, 6, 30, 31]
    assert chr_ == [0x30, 0x31, 0x32, 0x33, 0x10, 0x11, 0x20, 0x21] and nt == [0, 1, 0, 1]


def test_mmc3_scanline_irq():
    con = Console(cart(4, 128, 128))
    con.write(0xC000, 3)                                 # latch 3
    con.write(0xC001, 0)                                 # reload at the next clock
    con.write(0xE001, 0)                                 # enable
    con.write(0x2001, 0x18)                              # rendering on: clocks at dot 266 of lines 0-239
    con.set('p', 0x24)                                   # I set: the line stays asserted
    while con.u('frame_dot', 'I') < 3 * 341 + 266:
        assert con.u('irq_line') == 0
        con.step()
    assert con.u('irq_line') == 1                        # clock 1 reloads 3, clocks 2-4 count 2, 1, 0
    assert con.u('frame_dot', 'I') < 3 * 341 + 266 + 20
    con.write(0xE000, 0)                                 # acknowledge and disable
    assert con.u('irq_line') == 0


# ----------------------------------------------------------------------------------------------- MMC1

def mmc1_write(con, addr, value):
    for i in range(5):
        con.write(addr, (value >> i) & 1)


def mmc1_model(control, chr0, chr1, prg, banks16):
    """Board documentation: PRG 16 KB banks by mode, CHR 4 KB banks (8 KB mode ignores bit 0 of CHR0)."""
    mode = (control >> 2) & 3
    b = prg & 15
    if mode in (0, 1):
        lo, hi = b & ~1, (b & ~1) + 1
    elif mode == 2:
        lo, hi = 0, b
    else:
        lo, hi = b, banks16 - 1
    prg8 = [2 * lo, 2 * lo + 1, 2 * hi, 2 * hi + 1]
    if control & 0x10:
        c4 = [chr0, chr1]
    else:
        c4 = [chr0 & ~1, (chr0 & ~1) + 1]
    chr1k = [4 * c4[0] + i for i in range(4)] + [4 * c4[1] + i for i in range(4)]
    nt = {0: [0, 0, 0, 0], 1: [1, 1, 1, 1], 2: [0, 1, 0, 1], 3: [0, 0, 1, 1]}[control & 3]
    return prg8, chr1k, nt


@pytest.mark.parametrize('control', [0x00, 0x05, 0x0A, 0x0F, 0x12, 0x1C, 0x1F])
def test_mmc1_modes(control):
    con = Console(cart(1, 128, 128))
    mmc1_write(con, 0x8000, control)
    mmc1_write(con, 0xA000, 0x09)
    mmc1_write(con, 0xC000, 0x16)
    mmc1_write(con, 0xE000, 0x05)
    prg8, chr1k, nt = mmc1_model(control, 0x09, 0x16, 0x05, 8)
    got = pages(con)
    assert got[0] == [p % 16 for p in prg8] and got[1] == [c % 128 for c in chr1k] and got[2] == nt


def test_mmc1_reset_bit_and_power_on():
    con = Console(cart(1, 128, 128))
    assert pages(con)[0][2:] == [14, 15]                 # power-on: last 16 KB fixed at $C000
    con.write(0x8000, 1)
    con.write(0x8000, 1)
    con.write(0x8000, 0x80)                              # reset: shift cleared, PRG mode 3
    mmc1_write(con, 0xE000, 0x02)
    assert pages(con)[0] == [4, 5, 14, 15]


def test_mmc1_prg_ram_enable():
    con = Console(cart(1, 128, 128))
    con.write(0x6000, 0x5A)
    assert con.read(0x6000) == 0x5A
    mmc1_write(con, 0xE000, 0x10)                        # bit 4 disables PRG RAM
    con.write(0x6000, 0x11)
    assert con.read(0x6000) != 0x11
    mmc1_write(con, 0xE000, 0x00)
    assert con.read(0x6000) == 0x5A


def test_mmc1_synthetic_cart_switches_banks_mirroring_and_chr_ram():
    """The seed-generated MMC1 cart (the GPU parity case) does what it is for: it uploads its tiles into CHR RAM,
    switches the $8000 bank, flips the mirroring, keeps a CHR RAM tile animated and works in PRG RAM."""
    con = Console(synth.mmc1_cart(1))
    t, seen_prg, seen_nt, chr_sums = 82182, set(), set(), []
    for f in range(40):
        con.set('pad', [0x81, 0x40, 0x02, 0x90][f % 4])
        assert con.run_until(t) == 0
        t += 89342
        prg, _, nt = pages(con)
        seen_prg.add(prg[0])
        seen_nt.add(tuple(nt))
        chr_sums.append(int(con.rec[0x3C00:0x5C00].astype(np.int64).sum()))
    assert len(seen_prg) >= 4 and len(seen_nt) == 2
    assert chr_sums[10] > 0 and len(set(chr_sums[10:])) > 5
    assert con.rec[0x1C00:0x3C00].any()


# ------------------------------------------------------------------------------------------------ DMC

KBYTE = 8 * 54                                           # rate 15: 54 CPU cycles per bit


class Dmc:
    """The reference test's driver: 4-cycle instructions, the DMC serviced after each one."""

    def __init__(self):
        self.con = Console(cart(0, 16, 8))
        self.now = 1000
        self.stolen = 0
        self.con.lib.orc_dmc_reset(self.con.rec.ctypes.data, self.now)

    def write(self, a, v):
        self.con.write(a, v)

    def status(self):
        return self.con.read(0x4015)

    def event(self):
        return self.con.u('dmc_event', 'Q')

    def service(self, now, steal):
        return self.con.lib.orc_dmc_service(self.con.rec.ctypes.data, now, steal)

    def run(self, cycles):
        end = self.now + cycles
        while self.now < end:
            self.now += 4
            if self.now >= self.event():
                s = self.service(self.now, 1)
                self.now += s
                self.stolen += s


def test_dmc_power_on_is_silent():
    m = Dmc()
    assert m.status() == 0
    m.run(100 * KBYTE)
    assert m.stolen == 0 and m.event() == 2 ** 64 - 1


def test_dmc_seventeen_byte_sample():
    m = Dmc()
    m.run(3 * KBYTE + 100)
    m.write(0x4010, 0x0F)
    m.write(0x4013, 0x01)
    m.write(0x4015, 0x1F)
    assert m.status() == 0x10
    m.run(4)
    assert m.stolen == 4
    m.run(15 * KBYTE - 2 * 4)
    assert m.status() == 0x10
    m.run(2 * KBYTE)
    assert m.status() == 0x00 and m.stolen == 17 * 4
    m.run(10 * KBYTE)
    assert m.stolen == 17 * 4
    m.write(0x4015, 0x10)
    assert m.status() == 0x10


def test_dmc_restart_while_playing_and_stop():
    m = Dmc()
    m.write(0x4010, 0x0F)
    m.write(0x4013, 0x01)
    m.write(0x4015, 0x10)
    m.run(4 * KBYTE)
    assert 4 <= m.stolen // 4 <= 5
    m.write(0x4015, 0x10)
    m.run(4 * KBYTE)
    assert 8 <= m.stolen // 4 <= 9
    m.write(0x4015, 0x00)
    assert m.status() == 0
    before = m.stolen
    m.run(4 * KBYTE)
    assert m.stolen == before


def test_dmc_loop():
    m = Dmc()
    m.write(0x4010, 0x4F)
    m.write(0x4013, 0x00)
    m.write(0x4015, 0x10)
    m.run(100 * KBYTE)
    assert m.status() == 0x10 and 100 * 4 <= m.stolen <= 101 * 4


def test_dmc_rate_change_from_the_next_bit_clock():
    m = Dmc()
    m.write(0x4010, 0x4F)
    m.write(0x4015, 0x10)
    m.run(10 * KBYTE)
    m.write(0x4010, 0x40)
    m.run(8 * 428)
    before = m.stolen
    m.run(20 * 8 * 428)
    assert 19 * 4 <= m.stolen - before <= 21 * 4


def test_dmc_fast_forward_steals_nothing():
    m = Dmc()
    m.write(0x4010, 0x0F)
    m.write(0x4013, 0x01)
    m.write(0x4015, 0x10)
    start = m.now
    assert m.service(start, 0) == 0
    assert m.service(start + 10 * KBYTE, 0) == 0 and m.status() == 0x10
    assert m.service(start + 17 * KBYTE, 0) == 0 and m.status() == 0x00


# ----------------------------------------------------------------------------------------------- MMC2

def mmc2_con(chr_bytes=None):
    chr_ = bytes(32 * KB) if chr_bytes is None else bytes(chr_bytes)
    rom = bytearray(cart(9, 128, 32))
    rom[16 + 128 * KB:] = chr_
    return Console(bytes(rom))


def test_mmc2_registers_prg_and_chr_halves():
    """Power-on: both latches on the $FE bank; $A000 picks the 8 KB bank at $8000, the last three fixed; $B000-$E000
    the four 4 KB CHR banks, each half showing its latch's bank; $F000 bit 0: 0 vertical, 1 horizontal."""
    con = mmc2_con()
    assert list(con.mem('mreg', 8)[6:8]) == [1, 1]
    prg, _, _ = pages(con)
    assert prg[1:] == [13, 14, 15]
    for addr, v in ((0xA000, 5), (0xB000, 2), (0xC000, 3), (0xD000, 4), (0xE000, 6), (0xF000, 0)):
        con.write(addr, v)
    prg, chr_, nt = pages(con)
    assert prg == [5, 13, 14, 15]
    assert chr_ == [12, 13, 14, 15, 24, 25, 26, 27]            # latch 1 -> $FE banks 3 and 6 (4 KB -> 1 KB pages)
    assert nt == [0, 1, 0, 1]
    con.write(0xF000, 1)
    assert pages(con)[2] == [0, 0, 1, 1]
    con.write(0x9000, 7)                                        # $8000-$9FFF: no register
    assert pages(con)[0] == [5, 13, 14, 15]


def test_mmc2_cpu_driven_latch_flips():
    """$2006 and the $2007 address increments put VRAM addresses on the bus: $0FD0-$0FDF / $0FE0-$0FEF set latch 0
    to $FD / $FE, $1FD0-$1FEF latch 1 (patch:3196-3220)."""
    con = mmc2_con()
    for addr, v in ((0xB000, 2), (0xC000, 3), (0xD000, 4), (0xE000, 6)):
        con.write(addr, v)
    con.write(0x2006, 0x0F)
    con.write(0x2006, 0xD8)
    assert list(con.mem('mreg', 8)[6:8]) == [0, 1] and pages(con)[1][:4] == [8, 9, 10, 11]
    con.write(0x2006, 0x1F)
    con.write(0x2006, 0xCF)                                     # $1FCF: no flip
    assert list(con.mem('mreg', 8)[6:8]) == [0, 1]
    con.read(0x2007)                                            # the increment to $1FD0 flips latch 1 to $FD
    assert list(con.mem('mreg', 8)[6:8]) == [0, 0] and pages(con)[1][4:] == [16, 17, 18, 19]
    con.write(0x2006, 0x0F)
    con.write(0x2006, 0xE0)
    assert list(con.mem('mreg', 8)[6:8]) == [1, 0]


def test_mmc2_renderer_fetch_then_flip_along_the_line():
    """Background through half 0, latch 0 on $FE at the frame start. Bank $FD (2) holds opaque tiles, bank $FE (3)
    transparent ones. Nametable row 0 has tile $FD at slot 10 and $FE at slot 20: each fetch reads through the bank
    of the moment and then flips the latch (patch:1548-1551), so slots 11-20 are drawn from the $FD bank and every
    other slot, the two latch tiles' own left neighbours included, from the $FE bank; the latch carries over to the
    next line, which therefore looks the same."""
    chr_ = bytearray(32 * KB)
    for t in range(256):
        chr_[2 * 4 * KB + 16 * t: 2 * 4 * KB + 16 * t + 8] = b'\xff' * 8
    con = mmc2_con(chr_)
    for addr, v in ((0xB000, 2), (0xC000, 3), (0xD000, 4), (0xE000, 5)):
        con.write(addr, v)
    h = con.words('log', 16 + 512)
    h[:] = 0
    h[1] = 0x0A << 8                                            # background on, no left clip, pattern half 0
    h[3], h[4] = 0x0F0E0D0C, 0x17161514                         # the slot pages with both latches on $FE
    h[5] = 0b01000100
    h[6] = 0x0F | (0x21 << 8)                                   # backdrop $0F, colour 1 = $21
    h[14] = 2 | (3 << 8) | (4 << 16) | (5 << 24)
    h[15] = 1 | (1 << 8)
    con.set('log_n', 0, 'H')
    nt = con.mem('nt', 2048)
    nt[:] = 0
    nt[10], nt[20] = 0xFD, 0xFE
    con.mem('oam', 256)[:] = 0xFF
    pix = con.render_full()[0]
    want = np.full(256, 0x0F, np.uint8)
    want[88:168] = 0x21
    for y in (0, 1, 7):
        assert np.array_equal(pix[y], want), y


def resolve_frame(ctrl, mask, nt_cells, sprites, latches=(1, 1), events=(), mreg_latches=None):
    """A logged frame on an MMC2 console and its vblank resolve (oracle orc_mmc2_resolve): header with ctrl, mask,
    CHR banks $FD0 = 2, $FE0 = 3, $FD1 = 4, $FE1 = 5 and the given latches; nametable 0 cells {(row, col): tile},
    every other cell tile 0; sprites [(y, tile)] (the rest of OAM off screen); events [(kind, dot, value, aux)].
    Returns the latch registers and the CHR pages after the resolve."""
    con = mmc2_con()
    for addr, v in ((0xB000, 2), (0xC000, 3), (0xD000, 4), (0xE000, 5)):
        con.write(addr, v)
    if mreg_latches is not None:
        con.mem('mreg', 8)[6:8] = mreg_latches
    h = con.words('log', 16 + 512)
    h[:] = 0
    h[1] = ctrl | (mask << 8)
    h[5] = 0b01000100                                           # vertical mirroring: nametables 0, 1, 0, 1
    h[14] = 2 | (3 << 8) | (4 << 16) | (5 << 24)
    h[15] = latches[0] | (latches[1] << 8)
    for i, (kind, dot, value, aux) in enumerate(events):
        h[16 + 2 * i] = kind | (dot << 8) | (4 << 4)             # a 4-cycle instruction
        h[17 + 2 * i] = value | (aux << 8)
    con.set('log_n', len(events), 'H')
    nt = con.mem('nt', 2048)
    nt[:] = 0
    for (row, col), tile in nt_cells.items():
        nt[32 * row + col] = tile
    oam = con.mem('oam', 256)
    oam[:] = 0xFF
    for i, (y, tile) in enumerate(sprites):
        oam[4 * i:4 * i + 4] = (y, tile, 0, 100)
    con.lib.orc_mmc2_resolve(ptr(con.rec), con.cart_ptr())
    return [int(x) for x in con.mem('mreg', 8)[6:8]], pages(con)[1]


def test_mmc2_vblank_resolve_known_answers():
    """The latches a frame's own pattern fetches leave (patch:1790-1812: every line's background slots, then at the
    line's end the sprites of the next line, lines 0-239, from the latches of the frame's header; the hook of
    patch:1390-1402: a fetch at $0FD0-$0FDF / $0FE0-$0FEF sets latch 0 to the $FD / $FE bank, $1FDx / $1FEx latch 1).
    Each case is worked out by hand from those rules: which fetch of a trigger tile comes last in the frame."""
    bg0, bg1, spr1 = 0x00, 0x10, 0x08                           # ctrl: background table 0 or 1; sprites at $1000
    on = 0x18
    # background, half 0: a $FD tile on row 3 (lines 24-31) and a $FE tile on row 10 (lines 80-87): row 10 is
    # fetched last, so latch 0 ends on $FE (1); swapped, on $FD (0). Latch 1 keeps the header's value.
    assert resolve_frame(bg0, on, {(3, 5): 0xFD, (10, 7): 0xFE}, [], latches=(0, 0)) == (
        [1, 0], [12, 13, 14, 15, 16, 17, 18, 19])
    assert resolve_frame(bg0, on, {(3, 5): 0xFE, (10, 7): 0xFD}, [], latches=(1, 1)) == (
        [0, 1], [8, 9, 10, 11, 20, 21, 22, 23])
    # only $xFD0-$xFEF triggers: $FC and $FF tiles fetched after the $FE one change nothing
    assert resolve_frame(bg0, on, {(3, 5): 0xFE, (20, 1): 0xFC, (25, 9): 0xFF}, [], latches=(0, 0))[0] == [1, 0]
    # background and sprites both through half 1: the $FE tile on row 29 (lines 232-239) is fetched in every one of
    # those lines; a $FD sprite at y = 231 is fetched at the ends of lines 231-238 (for lines 232-239), before line
    # 239's background, so latch 1 ends on $FE; at y = 232 its last fetch is at the end of line 239 (for line 240),
    # after every background fetch, so latch 1 ends on $FD
    assert resolve_frame(bg1 | spr1, on, {(29, 4): 0xFE}, [(231, 0xFD)], latches=(0, 0))[0] == [0, 1]
    assert resolve_frame(bg1 | spr1, on, {(29, 4): 0xFE}, [(232, 0xFD)], latches=(0, 0))[0] == [0, 0]
    # sprites alone (background off, sprites on): the sprite fetches still run and flip latch 1
    assert resolve_frame(bg0 | spr1, 0x10, {}, [(100, 0xFE)], latches=(0, 0))[0] == [0, 1]
    # rendering off: no fetch at all; the latches are the header's, not what the registers held before
    assert resolve_frame(bg0 | spr1, 0x00, {(3, 5): 0xFD}, [(100, 0xFE)], latches=(1, 0), mreg_latches=(0, 1)) == (
        [1, 0], [12, 13, 14, 15, 16, 17, 18, 19])
    # a $2000 write in line 100 (NeSLE dot 100 * 341 + 150) moves the background to half 1: the $FD tile on row 3
    # sets latch 0, the $FE tile on row 20 (lines 160-167, after the write) sets latch 1
    ev = [(1, 100 * 341 + 150, bg1, 0)]
    assert resolve_frame(bg0, on, {(3, 5): 0xFD, (20, 9): 0xFE}, [], latches=(1, 0), events=ev)[0] == [0, 1]


def test_mmc2_synthetic_cart_flips_latches_while_rendering():
    """The seed-generated MMC2 cart's frames leave both latches changing from frame to frame (the vblank resolve)."""
    con = Console(synth.mmc2_cart(1))
    seen = set()
    target = 0
    for f in range(40):
        target += 89342
        con.run_until(target)
        seen.add(tuple(int(x) for x in con.mem('mreg', 8)[6:8]))
    assert len(seen) >= 3, seen
