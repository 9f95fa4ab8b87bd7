"""Known-answer tests of the oracle's PPU: registers, timing, the frame log and the line-replay renderer.

Pinned by the textbook PPU register model (t/v/x/w loopy registers written as named fields), the frame timing the
env is built on (rl/csrc/nes_machine.cuh:28-29: vblank at 241 * 341 + 1, 262 x 341 dots a frame), and restatements
of the reference's own PPU tests: the renderer pixel cases of third_party/nesle-extensions.patch:4413-4521 and the
SMB NMI frame-header case of patch:4249-4268 (the frame captured at the pre-render line starts from t).
"""
import numpy as np
import pytest

from helpers import Console
from rl import synth

VBLANK = 241 * 341 + 1
PRERENDER = 261 * 341 + 1
FRAME = 341 * 262
EV_SCROLL = 3
BIAS = 1024


def nrom(chr_bytes=None, vertical=True):
    prg = bytearray(16384)
    prg[0:4] = bytes((0xEA, 0x4C, 0x00, 0xC0))           # $C000: NOP; JMP $C000 (busy: no idle fast-forward)
    prg[0x3FFA:0x4000] = bytes((0x00, 0xC0, 0x00, 0xC0, 0x00, 0xC0))
    chr_ = bytearray(8192) if chr_bytes is None else bytearray(chr_bytes)
    return synth.ines(bytes(prg), bytes(chr_), 0, vertical=vertical)


def loopy(fine_y=0, nt=0, coarse_y=0, coarse_x=0):
    return (fine_y << 12) | (nt << 10) | (coarse_y << 5) | coarse_x


@pytest.fixture
def con():
    return Console(nrom())


# ------------------------------------------------------------------------------------------ registers

def test_scroll_and_address_latches(con):
    con.write(0x2000, 0x02)                              # nametable 2 into t
    assert con.u('t', 'H') == loopy(nt=2)
    con.write(0x2005, 0x7D)                              # first write: coarse x 15, fine x 5
    assert con.u('t', 'H') == loopy(nt=2, coarse_x=15) and con.u('fx') == 5 and con.u('w') == 1
    con.write(0x2005, 0x5E)                              # second write: coarse y 11, fine y 6
    assert con.u('t', 'H') == loopy(fine_y=6, nt=2, coarse_y=11, coarse_x=15) and con.u('w') == 0
    con.write(0x2006, 0xFF)                              # first write: bits 8-13 of t, bit 14 cleared
    assert con.u('t', 'H') == (0x3F << 8) | (loopy(fine_y=6, nt=2, coarse_y=11, coarse_x=15) & 0xFF)
    con.write(0x2006, 0x21)                              # second write: low byte, v = t
    assert con.u('t', 'H') == 0x3F21 and con.u('v', 'H') == 0x3F21 and con.u('w') == 0
    con.write(0x2005, 0x00)
    assert con.u('w') == 1
    con.read(0x2002)                                     # a status read resets the write toggle
    assert con.u('w') == 0


def test_vram_writes_mirroring_and_increment(con):
    con.write(0x2006, 0x28)
    con.write(0x2006, 0x05)                              # $2805 (vertical: same as $2005)
    con.write(0x2007, 0xAB)
    assert con.mem('nt', 2048)[5] == 0xAB and con.u('v', 'H') == 0x2806
    con.write(0x2000, 0x04)                              # increment 32
    con.write(0x2007, 0xCD)
    assert con.mem('nt', 2048)[6] == 0xCD and con.u('v', 'H') == 0x2826
    h = Console(nrom(vertical=False))                    # horizontal: $2400 is $2000
    h.write(0x2006, 0x24)
    h.write(0x2006, 0x00)
    h.write(0x2007, 0x11)
    h.write(0x2006, 0x28)
    h.write(0x2006, 0x00)
    h.write(0x2007, 0x22)
    assert h.mem('nt', 2048)[0] == 0x11 and h.mem('nt', 2048)[1024] == 0x22


def test_palette_mirrors_and_six_bits(con):
    for addr, val, slot in ((0x3F10, 0x7F, 0x00), (0x3F14, 0x21, 0x04), (0x3F01, 0x15, 0x01), (0x3F31, 0x0A, 0x11)):
        con.write(0x2006, addr >> 8)
        con.write(0x2006, addr & 0xFF)
        con.write(0x2007, val)
        assert con.mem('pal', 32)[slot] == val & 0x3F, hex(addr)


def test_ppudata_read_buffer(con):
    con.write(0x2006, 0x20)
    con.write(0x2006, 0x00)
    for v in (0x10, 0x20, 0x30):
        con.write(0x2007, v)
    con.write(0x2006, 0x20)
    con.write(0x2006, 0x00)
    stale = con.read(0x2007)                             # the buffer, then $2000's byte into it
    assert con.read(0x2007) == 0x10 and con.read(0x2007) == 0x20 and stale == 0
    con.write(0x2006, 0x3F)
    con.write(0x2006, 0x01)
    con.write(0x2007, 0x2A)
    con.write(0x2006, 0x3F)
    con.write(0x2006, 0x01)
    assert con.read(0x2007) == 0x2A                      # palette reads are immediate
    assert con.u('read_buf') == con.mem('nt', 2048)[0x301]   # ... and buffer the nametable byte under them


def test_controller_port():
    con = Console(nrom())
    con.set('pad', 0b10110010)
    con.write(0x4016, 1)
    assert [con.read(0x4016) for _ in range(3)] == [0x40] * 3      # strobe high: bit 0 (A) again and again
    con.write(0x4016, 0)
    bits = [con.read(0x4016) & 1 for _ in range(10)]
    assert bits == [0, 1, 0, 0, 1, 1, 0, 1, 1, 1]                  # A first ... Right last, then 1s


def test_oam_dma_copies_a_page_and_stalls(con):
    ram = con.ram()
    ram[0x200:0x300] = np.arange(256, dtype=np.uint8)[::-1]
    for start_cycles in (7, 8):
        con.set('cycles', start_cycles, 'Q')
        con.ram()[0x300:0x303] = (0x8D, 0x14, 0x40)      # STA $4014 with A = 2
        con.set('a', 2)
        con.set('pc', 0x0300, 'H')
        cyc, fault = con.step()
        after = start_cycles + 4
        assert fault == 0 and cyc == 4 + 513 + (after & 1)
        assert np.array_equal(con.mem('oam', 256), ram[0x200:0x300])


# ----------------------------------------------------------------------------------------------- timing

def test_vblank_flag_and_nmi_timing(con):
    """Stepping the NOP loop instruction by instruction: the vblank flag is up exactly from dot 241 * 341 + 1, the
    NMI is taken by the next step, and the flags drop at the pre-render dot 261 * 341 + 1."""
    con.write(0x2000, 0x80)                              # NMI on vblank
    con.set('p', 0x24)
    seen = False
    while con.u('frame_dot', 'I') < VBLANK + 30:
        before = con.u('frame_dot', 'I')
        cyc, fault = con.step()
        assert fault == 0
        dot = con.u('frame_dot', 'I')
        assert bool(con.u('status') & 0x80) == (dot >= VBLANK), (before, dot)
        if dot >= VBLANK and not seen:
            seen = True
            assert con.u('nmi_pending') == 1
            cyc, fault = con.step()                      # NMI entry (7) + NOP (2)
            assert cyc == 9 and con.u('nmi_pending') == 0 and con.u('sp') == 0xFD - 3
    while con.u('frame_dot', 'I') < PRERENDER + 30:
        dot0 = con.u('frame_dot', 'I')
        con.step()
        dot = con.u('frame_dot', 'I')
        if dot0 < PRERENDER <= dot:
            assert con.u('status') & 0xE0 == 0
        elif dot < PRERENDER:
            assert con.u('status') & 0x80
    assert con.run_until(FRAME) == 0 and con.u('frame', 'I') == 1


def test_run_until_stops_at_the_first_event_at_or_after_the_target(con):
    assert con.run_until(VBLANK) == 0
    dot = con.u('frame_dot', 'I')
    assert VBLANK <= dot < VBLANK + 3 * 7 and con.u('status') & 0x80


def test_status_read_clears_vblank(con):
    assert con.run_until(VBLANK) == 0
    v = con.read(0x2002)
    assert v & 0x80 and con.u('status') & 0x80 == 0


def test_frame_header_starts_from_t_not_ppuctrl(con):
    """SMB's NMI: $2000 = $10 (status bar on nametable 0), VRAM update ending $2006 = $3F00, $0000, then the
    playfield nametable selected in PPUCTRL; the frame captured at the pre-render line starts from t."""
    assert con.run_until(VBLANK) == 0
    con.write(0x2000, 0x10)
    con.write(0x2000, 0x15)
    for b in (0x3F, 0x00, 0x00, 0x00):
        con.write(0x2006, b)
    assert con.run_until(PRERENDER) == 0
    h = con.words('log', 16)
    assert con.u('ctrl') == 0x15 and h[1] & 0xFF == 0x15 and h[2] >> 16 == 0
    con.write(0x2000, 0x91)                              # NMI exit without $2006: t keeps nametable 1
    assert con.run_until(FRAME + PRERENDER) == 0
    h = con.words('log', 16)
    assert h[1] & 0xFF == 0x91 and (h[2] >> 16 >> 10) & 3 == 1


# --------------------------------------------------------------------------------------------- renderer

class Picture:
    """A console whose logged frame is set by hand: header, nametables, OAM, CHR."""

    def __init__(self, mask, ctrl=0, chr_bytes=None):
        self.chr = bytearray(8192) if chr_bytes is None else bytearray(chr_bytes)
        self.con = Console(nrom(self.chr))
        self.chr_view = self.con.rom[16 + 16384:16 + 16384 + 8192]
        self.h = self.con.words('log', 16 + 512)
        self.h[:] = 0
        self.h[1] = ctrl | (mask << 8)
        self.h[3] = 0x03020100                           # CHR slots 0-7 -> pages 0-7
        self.h[4] = 0x07060504
        self.h[5] = 0b01000100                           # vertical arrangement: 0, 1, 0, 1
        self.con.set('log_n', 0, 'H')
        self.nt = self.con.mem('nt', 2048)
        self.oam = self.con.mem('oam', 256)
        self.oam[:] = 0xFF                               # every sprite below the screen

    def palette(self, i, v):
        w = self.h[6 + i // 4]
        self.h[6 + i // 4] = (int(w) & ~(0xFF << (8 * (i % 4)))) | (v << (8 * (i % 4)))

    def event(self, time, kind, value, aux=0):
        n = self.con.u('log_n', 'H')
        self.h[16 + 2 * n] = ((time + BIAS) & 0xFFFFFF) | (kind << 24)
        self.h[17 + 2 * n] = value | (aux << 8)
        self.con.set('log_n', n + 1, 'H')
        self.h[0] = n + 1

    def render(self):
        pix, emph = self.con.render_full()
        return pix


def test_background_tile_top_left_and_left_clip():
    p = Picture(mask=0x0A)
    p.chr_view[0x0010] = 0x80                            # tile 1, row 0: leftmost pixel colour 1
    p.nt[0] = 0x01
    p.palette(1, 0x21)
    pix = p.render()
    assert pix[0, 0] == 0x21 and pix[0, 1] == 0x00 and pix[1, 0] == 0x00 and pix[0, 8] == 0x00
    p.h[1] = 0x08 << 8                                   # left column hidden: the backdrop
    assert p.render()[0, 0] == 0x00


def test_sprite_at_oam_y_is_drawn_from_the_next_line():
    p = Picture(mask=0x14)
    p.chr_view[0x0020] = 0x80                            # tile 2, row 0: leftmost pixel colour 1
    p.palette(0x11, 0x16)
    p.oam[0:4] = (9, 2, 0, 12)
    pix = p.render()
    assert pix[10, 12] == 0x16 and pix[9, 12] == 0x00 and pix[10, 13] == 0x00


def test_mid_frame_scroll_write_from_the_log():
    p = Picture(mask=0x0A)
    for row in range(8):
        p.chr_view[0x0010 + row] = 0xFF                  # tile 1: every pixel colour 1
    for col in range(0, 32, 2):
        for tile_row in range(30):
            p.nt[tile_row * 32 + col] = 0x01
    p.palette(1, 0x21)
    p.event(100 * 341 + 240 + 3 * 4, EV_SCROLL, 8, 0)    # $2005 = 8 by a 4-cycle store from dot 240 of line 100
    pix = p.render()
    assert pix[50, 0] == 0x21 and pix[50, 8] == 0x00
    assert pix[100, 0] == 0x21 and pix[100, 8] == 0x00
    assert pix[101, 0] == 0x00 and pix[101, 8] == 0x21
    assert pix[200, 0] == 0x00 and pix[200, 8] == 0x21


def test_sprite_priority_and_eight_per_line():
    p = Picture(mask=0x1E)
    for row in range(8):
        p.chr_view[0x0010 + row] = 0xFF                  # tile 1 opaque colour 1
        p.chr_view[0x0020 + row] = 0xFF                  # tile 2: colour 3 (both planes)
        p.chr_view[0x0028 + row] = 0xFF
    p.nt[:960] = 0x01                                    # opaque background everywhere
    p.palette(1, 0x01)
    p.palette(0x13, 0x33)                                # sprite palette 0 colour 3
    p.palette(0x17, 0x37)                                # sprite palette 1 colour 3
    p.oam[0:4] = (49, 2, 0x01, 100)                      # in front, palette 1
    p.oam[4:8] = (49, 2, 0x20, 120)                      # behind the background
    pix = p.render()
    assert pix[50, 100] == 0x37 and pix[50, 120] == 0x01
    for i in range(9):                                   # nine sprites on one line: only the first eight show
        p.oam[4 * i:4 * i + 4] = (79, 2, 0x00, 8 + 16 * i)
    pix = p.render()
    assert all(pix[80, 8 + 16 * i] == 0x33 for i in range(8)) and pix[80, 8 + 16 * 8] == 0x01


def test_greyscale_and_emphasis():
    p = Picture(mask=0x0A | 0x01 | 0xE0)
    p.chr_view[0x0010] = 0x80
    p.nt[0] = 0x01
    p.palette(1, 0x2D)
    pix, emph = p.con.render_full()
    assert pix[0, 0] == 0x2D & 0x30 and (emph == 7).all()


def test_sprite0_hit_dot():
    p = Picture(mask=0x1E)
    for row in range(8):
        p.chr_view[0x0010 + row] = 0xFF
    p.nt[:960] = 0x01
    p.oam[0:4] = (30, 1, 0, 40)                          # sprite 0 from line 31, x 40, over opaque background
    assert p.con.lib.orc_sprite0_scan(p.con.rec.ctypes.data, p.con.cart_ptr()) == 31 * 341 + 40 + 1
    p.oam[3] = 255                                       # x = 255 never hits
    assert p.con.lib.orc_sprite0_scan(p.con.rec.ctypes.data, p.con.cart_ptr()) == 0x7FFFFFFF
    p.oam[3] = 2                                         # left 8 pixels clipped for sprites: first hit at x 8
    p.h[1] = 0x18 << 8
    assert p.con.lib.orc_sprite0_scan(p.con.rec.ctypes.data, p.con.cart_ptr()) == 31 * 341 + 8 + 1
