"""Known-answer tests of the oracle's PPU: registers, timing, the frame log and the line-replay renderer.

Pinned by the textbook PPU register model (t/v/x/w loopy registers written as named fields), the frame timing the
env is built on (rl/csrc/nes_machine.cuh:28-29: vblank at 241 * 341 + 1, 262 x 341 dots a frame), and restatements
of the reference's own PPU tests: the renderer pixel cases of third_party/nesle-extensions.patch:4413-4521 and the
SMB NMI frame-header case of patch:4249-4268 (the frame captured at the pre-render line starts from t).
"""
import ctypes

import numpy as np
import pytest

from helpers import Console
from rl import synth

VBLANK = 241 * 341 + 1
PRERENDER = 261 * 341 + 1
FRAME = 341 * 262


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

VFLAG = VBLANK - 12                                      # the replay's $2002 flag: 12 dots before NMI (patch:1940-1945)
SCLR = PRERENDER - 12


def test_vblank_flag_nmi_and_status_clear_timing(con):
    """Stepping the NOP loop instruction by instruction: $2002 bit 7 is up from 241 * 341 + 1 - 12, the NMI is
    raised at 241 * 341 + 1 and taken by the next step, and the flags drop at the pre-render dot - 12."""
    con.write(0x2000, 0x80)                              # NMI on vblank
    con.set('p', 0x24)
    seen = False
    while con.u('frame_dot', 'I') < VBLANK + 30:
        cyc, fault = con.step()
        assert fault == 0
        dot = con.u('frame_dot', 'I')
        assert bool(con.u('status') & 0x80) == (dot >= VFLAG), dot
        assert bool(con.u('nmi_pending')) == (dot >= VBLANK and not seen), dot
        if dot >= VBLANK and not seen:
            seen = True
            cyc, fault = con.step()                      # NMI entry (7) + NOP (2)
            assert cyc == 9 and con.u('nmi_pending') == 0 and con.u('sp') == 0xFD - 3
    while con.u('frame_dot', 'I') < PRERENDER + 30:
        dot0 = con.u('frame_dot', 'I')
        con.step()
        dot = con.u('frame_dot', 'I')
        if dot >= SCLR:
            assert con.u('status') & 0xE0 == 0
        else:
            assert con.u('status') & 0x80
    assert con.run_until(FRAME) == 0 and con.u('frame', 'I') == 1


def test_nmi_fires_even_when_a_read_took_the_flag(con):
    """A $2002 read between the flag (dot 82170) and NMI (82182) clears bit 7, and the NMI still comes."""
    con.write(0x2000, 0x80)
    con.set('p', 0x24)
    while con.u('frame_dot', 'I') < VFLAG:
        con.step()
    assert con.u('frame_dot', 'I') < VBLANK and con.read(0x2002) & 0x80 and con.u('status') & 0x80 == 0
    while con.u('frame_dot', 'I') < VBLANK:
        con.step()
    assert con.u('nmi_pending') == 1


def test_kook_frames_alternate_and_drop_the_last_pre_render_dot(con):
    """Every other frame's pre-render line is a dot short: the header of every second frame captured carries the
    kook bit, and a step across that frame's wrap lands one dot further."""
    kooks = []
    for f in range(1, 6):
        assert con.run_until(f * FRAME) == 0
        kooks.append((int(con.words('log', 16)[5]) >> 8) & 1)
    assert kooks == [0, 1, 0, 1, 0]
    for short in (0, 1):
        c2 = Console(nrom())
        c2.set('frame_dot', FRAME - 4, 'I')
        c2.set('log_flags', 2 * short)
        c2.set('pc', 0xC000, 'H')
        cyc, fault = c2.step()                           # NOP: 2 cycles, 6 dots, across the wrap
        assert cyc == 2 and c2.u('frame', 'I') == 1 and c2.u('frame_dot', 'I') == 2 + short
        assert c2.u('log_flags') & 2 == 0                # the short frame has ended


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
#
# The replay grid (third_party/nesle-extensions.patch:900-1830): a write by an instruction that starts at NeSLE frame
# dot d with c cycles lands at position p = d + 11 + 3c - (l * 341 - 16) of line l; the line's tile slots are drawn
# in steps of 8 positions up to p / 8 before it (slot k's tile is fetched there and shows 16 pixels later, at pixels
# 8(k - 2)..8(k - 2) + 7), a $2007 write draws nothing first, and what is left of the line is drawn at position 272.

EV = dict(ctrl=1, mask=2, scroll=3, addr=4, data=5, pal=6, chr=7, mirror=8, mmc2=9, dread=10)


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

    def event(self, line, dot, kind, value, aux=0, cycles=4):
        """A write by a `cycles`-cycle instruction that starts at dot `dot` of line `line` (NeSLE's grid)."""
        n = self.con.u('log_n', 'H')
        d = line * 341 + dot if line >= 0 else PRERENDER - 1 + dot
        self.h[16 + 2 * n] = EV[kind] | (cycles << 4) | (d << 8)
        self.h[17 + 2 * n] = value | (aux << 8)
        self.con.set('log_n', n + 1, 'H')
        self.h[0] = n + 1

    def render(self):
        pix, emph = self.con.render_full()
        return pix

    def opaque_tile(self, tile=1, planes=(0,)):
        for row in range(8):
            for pl in planes:
                self.chr_view[16 * tile + 8 * pl + row] = 0xFF


def stripes(p):
    """Tile 1 (opaque colour 1) in the even columns of both nametables, tile 0 (transparent) in the odd ones,
    palette 1 = $21, backdrop $0F."""
    p.opaque_tile(1)
    for col in range(0, 32, 2):
        for tile_row in range(30):
            p.nt[tile_row * 32 + col] = 0x01
            p.nt[1024 + tile_row * 32 + col] = 0x01
    p.palette(0, 0x0F)
    p.palette(1, 0x21)


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


def test_tall_sprites_take_the_tile_pair_and_flip_as_one():
    """8x16 sprites (ctrl bit 5): tile byte 3 selects the pattern table at $1000 (bit 0) and the tiles 2 (rows 0-7)
    and 3 (rows 8-15). Tile 2's row 0 has its leftmost pixel set, tile 3's row 7 its rightmost. Drawn from line
    y + 1: unflipped, line 10 shows the first and line 25 the second; flipped vertically the 16 rows run backwards
    across both tiles (line 10 shows tile 3's row 7); flipped horizontally the leftmost pixel moves to x + 7."""
    def pic(attr):
        p = Picture(mask=0x14, ctrl=0x20)
        p.chr_view[0x1000 + 2 * 16 + 0] = 0x80
        p.chr_view[0x1000 + 3 * 16 + 7] = 0x01
        p.palette(0x11, 0x16)
        p.oam[0:4] = (9, 3, attr, 12)
        return p.render()
    pix = pic(0x00)
    assert pix[10, 12] == 0x16 and pix[25, 19] == 0x16
    assert (pix[10] == 0x16).sum() == 1 and (pix[25] == 0x16).sum() == 1 and (pix[11:25] == 0x16).sum() == 0
    pix = pic(0x80)
    assert pix[10, 19] == 0x16 and pix[25, 12] == 0x16
    assert (pix[10] == 0x16).sum() == 1 and (pix[25] == 0x16).sum() == 1 and (pix[11:25] == 0x16).sum() == 0
    pix = pic(0x40)
    assert pix[10, 19] == 0x16 and pix[25, 12] == 0x16
    assert (pix[26] == 0x16).sum() == 0 and (pix[9] == 0x16).sum() == 0


def test_scroll_written_in_hblank_takes_effect_on_the_next_line():
    """$2005 = 8 by a 4-cycle store from dot 240 of line 100: position 240 + 39 = 279 is past the line's pixels
    (272), so line 100 keeps the old scroll and the horizontal copy at its end brings coarse x 1 to line 101."""
    p = Picture(mask=0x0A)
    stripes(p)
    p.event(100, 240, 'scroll', 8, 0)
    pix = p.render()
    for y in (50, 100):
        assert pix[y, 0] == 0x21 and pix[y, 8] == 0x0F
    for y in (101, 200):
        assert pix[y, 0] == 0x0F and pix[y, 8] == 0x21


def test_mask_write_mid_line_cuts_to_the_backdrop_at_its_tile():
    """$2001 = 0 by a 4-cycle store from dot 100 of line 50 lands at position 100 + 39 = 139: slots 0..16 are drawn
    before it (pixels 0..119 from the background), the rest of the line and every later line is the backdrop."""
    p = Picture(mask=0x0A)
    p.opaque_tile(1)
    p.nt[:960] = 0x01
    p.palette(0, 0x0F)
    p.palette(1, 0x21)
    p.event(50, 100, 'mask', 0x00)
    pix = p.render()
    assert (pix[49] == 0x21).all()
    assert (pix[50, :120] == 0x21).all() and (pix[50, 120:] == 0x0F).all()
    assert (pix[51:] == 0x0F).all()


def test_fine_x_written_mid_line_shifts_the_rest_of_it():
    """A first $2005 write of 3 (coarse x 0, fine x 3) from dot 100 of line 60: slots 0..16 keep fine x 0; from
    pixel 120 on each pixel x shows background column x + 3; line 61 takes coarse x 0 from t and keeps fine x 3."""
    p = Picture(mask=0x0A)
    stripes(p)
    p.event(60, 100, 'scroll', 0x03, 0)
    pix = p.render()
    col = np.arange(256)
    want = lambda shift: np.where(((col + shift) // 8) % 2 == 0, 0x21, 0x0F)
    assert np.array_equal(pix[59], want(0))
    assert np.array_equal(pix[60, :120], want(0)[:120]) and np.array_equal(pix[60, 120:], want(3)[120:])
    assert np.array_equal(pix[61], want(3))


def test_address_written_mid_line_moves_the_fetches_at_once():
    """Rows 0-14 of the nametable opaque, rows 15-29 transparent. $2006 = $21 from dot 90 and $E0 from dot 102 of
    line 40 (4-cycle stores, positions 129 and 141): the second write sets v = $21E0 (row 15, fine y 2) after slot
    16, so background columns 0..16 (pixels 0..135) come from row 5 and the rest from row 15; line 41 stays in
    row 15."""
    p = Picture(mask=0x0A)
    p.opaque_tile(1)
    p.nt[:15 * 32] = 0x01
    p.palette(0, 0x0F)
    p.palette(1, 0x21)
    p.event(40, 90, 'addr', 0x21, 0)
    p.event(40, 102, 'addr', 0xE0, 1)
    pix = p.render()
    assert (pix[39] == 0x21).all()
    assert (pix[40, :136] == 0x21).all() and (pix[40, 136:] == 0x0F).all()
    assert (pix[41] == 0x0F).all()


def test_palette_write_draws_nothing_first():
    """A $2007 palette write (colour 1 = $16) from dot 100 of line 70 triggers no drawing: the whole line is drawn
    at its end with the new colour. On line 75 a $2000 write from dot 50 (position 89) first draws slots 0..10, so
    pixels 0..71 keep the old colour."""
    p = Picture(mask=0x0A)
    p.opaque_tile(1)
    p.nt[:960] = 0x01
    p.nt[1024:1024 + 960] = 0x01                         # (the write's own address increment moves the fetches)
    p.palette(1, 0x21)
    p.event(70, 100, 'pal', 0x16, 1)
    p.event(72, 100, 'pal', 0x21, 1)
    p.event(75, 50, 'ctrl', 0x00)
    p.event(75, 100, 'pal', 0x16, 1)
    pix = p.render()
    assert (pix[69] == 0x21).all() and (pix[70] == 0x16).all() and (pix[72] == 0x21).all()
    assert (pix[75, :72] == 0x21).all() and (pix[75, 72:] == 0x16).all()
    assert (pix[76] == 0x16).all()


def test_greyscale_applies_only_while_rendering():
    """Greyscale keeps bits 4-5 of each colour while the background or sprites are on; with both off the backdrop
    keeps all six bits ($2D stays $2D)."""
    p = Picture(mask=0x0A | 0x01 | 0xE0)
    p.chr_view[0x0010] = 0x80
    p.nt[0] = 0x01
    p.palette(1, 0x2D)
    pix, emph = p.con.render_full()
    assert pix[0, 0] == 0x2D & 0x30 and (emph == 7).all()
    q = Picture(mask=0x01)
    q.palette(0, 0x2D)
    assert (q.render() == 0x2D).all()


def test_emphasis_is_the_mask_at_the_end_of_the_line():
    """Emphasis bits from $2001 written from dot 100 of line 90 (during its pixels) show on line 90 itself; written
    from dot 300 of line 80 (after position 272) they start on line 81."""
    p = Picture(mask=0x0A)
    p.event(80, 300, 'mask', 0x2A)
    p.event(90, 100, 'mask', 0x4A)
    pix, emph = p.con.render_full()
    assert emph[80] == 0 and emph[81] == 1 and emph[89] == 1 and emph[90] == 2


def test_sprite_line_latched_while_sprites_were_on_is_drawn_when_they_come_back():
    """Sprite 1 covers lines 100-107. Sprites are on at the end of line 99 (its line is latched) and turned off by
    a write from dot 10 of line 100, so line 100 draws no sprite and keeps the latched line pending; turned on again
    from dot 10 of line 120, line 120 draws that stale line (x 40) and line 121 nothing."""
    p = Picture(mask=0x1E)
    p.opaque_tile(2)
    p.palette(0x11, 0x16)
    p.oam[4:8] = (99, 2, 0, 40)
    p.event(100, 10, 'mask', 0x0E)
    p.event(120, 10, 'mask', 0x1E)
    pix = p.render()
    assert pix[99, 40] == 0x00 and pix[100, 40] == 0x00 and pix[110, 40] == 0x00
    assert (pix[120, 40:48] == 0x16).all() and pix[120, 39] == 0x00 and pix[121, 40] == 0x00


def test_rendering_turned_on_during_the_prefetch_shifts_the_line():
    """Background turned on by a 2-cycle write from dot 326 of the pre-render line (replay time -4, inside line 0's
    lead-in, position 18): v = t is not done (rendering was off), slots 0-1 are drawn with rendering off and still
    advance the output position by 16, and the shift registers start empty, so line 0 shows background column j at
    pixel 32 + 8j."""
    p = Picture(mask=0x00)
    stripes(p)
    p.event(-1, 326, 'mask', 0x0A, cycles=2)
    pix = p.render()
    col = np.arange(256)
    want = np.where(col < 32, 0x0F, np.where(((col - 32) // 8) % 2 == 0, 0x21, 0x0F))
    assert np.array_equal(pix[0], want)


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


# ------------------------------------------------------------------------------------------- sprite 0

def sprite0(p):
    hit = ctypes.c_int(0)
    dot = p.con.lib.orc_sprite0_hit(p.con.rec.ctypes.data, p.con.cart_ptr(), ctypes.byref(hit))
    return dot, hit.value


def test_sprite0_hit_dot():
    """Sprite 0 from line 31 at x 40 over opaque background: pixel 40 is drawn (with the slot the pending check
    adds) and left of p - 16 from line position 57, so a 4-cycle $2002 read that ends there, i.e. starts at NeSLE
    dot 31 * 341 - 16 + 57 - 12 - 11, sees the flag. x 255 never hits: the answer is then the end of sprite 0's
    lines (line 46, position 256); sprite 0 below the picture gives no check at all."""
    p = Picture(mask=0x1E)
    p.opaque_tile(1)
    p.nt[:960] = 0x01
    p.oam[0:4] = (30, 1, 0, 40)
    assert sprite0(p) == (31 * 341 - 16 + 57 - 23, 1)
    p.oam[3] = 255
    assert sprite0(p) == (46 * 341 + 256 - 11, 0)
    p.oam[0] = 239
    assert sprite0(p) == (0, 0)


def test_sprite0_hit_left_column_follows_the_background_clip_only():
    """Sprite 0 at x 2. With the background's left column hidden the first opaque background pixel under it is 8,
    seen from position 32 (slot 4 drawn, 8 < 32 - 16); with it shown the hit is at x 2 from position 19 even though
    the sprites' own left column is hidden (FCEUmm's check looks at the background only)."""
    p = Picture(mask=0x18)
    p.opaque_tile(1)
    p.nt[:960] = 0x01
    p.oam[0:4] = (30, 1, 0, 2)
    assert sprite0(p) == (31 * 341 - 16 + 32 - 23, 1)
    p.h[1] = 0x1A << 8
    assert sprite0(p) == (31 * 341 - 16 + 19 - 23, 1)


def test_bit_2002_polling_sees_the_hit_at_its_dot():
    """A BIT $2002 / BVC loop (7 cycles) spinning on bit 6 with sprite 0 at line 31, x 40: the first BIT that reads
    the flag is the first one that starts at or after the hit dot (31 * 341 + 18), and none before it does."""
    prg = bytearray(16384)
    prg[0:5] = bytes((0x2C, 0x02, 0x20, 0x50, 0xFB))     # $C000: BIT $2002; BVC $C000
    prg[5:8] = bytes((0x4C, 0x05, 0xC0))                 # $C005: JMP $C005
    prg[0x3FFA:0x4000] = bytes((0x00, 0xC0, 0x00, 0xC0, 0x00, 0xC0))
    chr_ = bytearray(8192)
    for row in range(8):
        chr_[0x10 + row] = 0xFF
    con = Console(synth.ines(bytes(prg), bytes(chr_), 0, vertical=True))
    con.set('p', 0x24)
    con.write(0x2001, 0x1E)
    con.mem('nt', 2048)[:960] = 0x01
    oam = con.mem('oam', 256)
    oam[:] = 0xFF
    oam[0:4] = (30, 1, 0, 40)
    assert con.run_until(FRAME) == 0                     # through a pre-render line: the frame's check is scheduled
    hit_dot = 31 * 341 + 18
    starts = []
    while con.u('pc', 'H') != 0xC005:
        if con.u('pc', 'H') == 0xC000:
            starts.append(con.u('frame_dot', 'I'))
        cyc, fault = con.step()
        assert fault == 0 and con.u('frame', 'I') == 1
    assert starts[-1] >= hit_dot and starts[-2] < hit_dot


# --------------------------------------------------------------------------- what the parity carts exercise

def line_landings(con):
    """(line, position) of every logged write of the console's frame that lands while a visible line is drawn:
    position = the instruction's end on the replay grid minus the line's start (16 dots before its dot 0)."""
    h = con.words('log', 16 + 512)
    n = min(con.u('log_n', 'H'), 256)
    kook = (int(h[5]) >> 8) & 1
    out = []
    for i in range(n):
        w0 = int(h[16 + 2 * i])
        kind, cyc, dot = w0 & 15, (w0 >> 4) & 15, (w0 >> 8) & 0x1FFFF
        if kind in (EV['data'], EV['pal']):
            continue
        t = dot - FRAME + 11 + kook if dot >= PRERENDER else dot + 11
        end = t + 3 * cyc
        line = (t + 16) // 341
        pos = end - (line * 341 - 16)
        if 0 <= line < 240 and 17 <= pos < 272:
            out.append((line, pos))
    return out


@pytest.mark.parametrize('make', [lambda: synth.mmc3_cart(1), lambda: synth.smb_like_cart(1)], ids=['mmc3', 'smb'])
def test_parity_carts_split_lines_mid_line_and_hit_sprite0(make):
    """The seed-generated carts of the GPU parity tests draw frames the textbook line-start model would get wrong:
    writes that land while a visible line is being drawn, and sprite-0 hits the CPU waits on."""
    con = Console(make())
    mid, hits = 0, 0
    for f in range(1, 41):
        con.set('pad', [0x81, 0x40, 0x02, 0xC0, 0x10][f % 5])
        assert con.run_until(f * FRAME + VBLANK) == 0
        mid += len(line_landings(con))
        hit = ctypes.c_int(0)
        con.lib.orc_sprite0_hit(con.rec.ctypes.data, con.cart_ptr(), ctypes.byref(hit))
        hits += hit.value
    assert mid >= 10 and hits >= 10, (mid, hits)


def test_vblank_io_cart_writes_every_ppu_register_in_vblank():
    """The vblank I/O cart's NMI, stepped one instruction at a time on the oracle over 24 frames: by the time it
    counts its frame, the OAM holds the sprite it wrote through $2003/$2004 (and, every eighth frame, the four bytes
    from $FE on, wrapping into sprite 0), the palette entry FRAMES & 31 (its $3F10 mirror folded) holds the byte
    written through $2006/$2007, the nametable column holds its six bytes 32 apart (written through the $2007 mirror
    $2FFF) and the byte of the indexed store below them, and a nested NMI has been taken exactly in the frames whose
    counter is a multiple of 4 (NMI turned off and on while the vblank flag was up)."""
    con = Console(synth.vblank_io_cart(1))
    ram = con.ram()
    checked, nested_frames = 0, 0
    for _ in range(400000):
        depth = int(ram[synth.NMI_DEPTH])
        con.step()
        if depth == 0 and ram[synth.NMI_DEPTH] == 1 and ram[synth.FRAMES] >= 2:   # the first NMI's INC NMI_DEPTH
            f, px, py, cnt, pad, nested = (int(ram[k]) for k in (synth.FRAMES, synth.PX, synth.PY, synth.CNT_LO,
                                                                 synth.PAD, synth.NESTED))
            while ram[synth.FRAMES] == f:
                con.step()
            oam, pal, nt = con.mem('oam', 256), con.mem('pal', 32), con.mem('nt', 2048)
            s = ((f & 15) + 2) * 4
            assert list(oam[s:s + 4]) == [(py + 16) & 0xFF, cnt, f & 0xE3, px ^ 0x55], f
            if f % 8 == 0:
                assert list(oam[[0xFE, 0xFF, 0, 1]]) == [0x21 ^ f, 0x40 ^ f, 0x30 ^ f, f], f
            i = f & 31
            assert pal[i & 0x0F if (i & 0x13) == 0x10 else i] == (cnt ^ pad) & 0x3F, f
            base = 1024 + (f & 31)                          # nametable 1 or 3: one under vertical mirroring
            assert [int(nt[base + 32 * k]) for k in range(6)] == [(6 - k) ^ f for k in range(6)], f
            assert nt[base + 192] == pad, f
            took = int(ram[synth.NESTED]) - nested
            assert took == (1 if f % 4 == 0 else 0), f
            nested_frames += took
            checked += 1
            if checked == 24:
                break
    assert checked == 24 and nested_frames == 6, (checked, nested_frames)
