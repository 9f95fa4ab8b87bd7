"""Seed-generated workloads: synthetic NES cartridges (iNES images) and SMB-style RAM trajectories.

The reference ships no ROMs (its README names the commercial carts it trains on), so the benchmark configs use
cartridges generated here from a seed:

* ``nrom_cart(seed)`` - NROM-128: 16 KB PRG of generated 6502 code (reset init, an NMI handler doing OAM DMA via
  $4014 and nametable writes via $2006/$2007, a main loop reading $4016 and branching on the pad bits, RAM
  counters and seeded arithmetic blocks) and 8 KB CHR of uniform-random 2bpp tiles.
* ``mmc3_cart(seed)`` - MMC3: 256 KB PRG / 128 KB CHR. The main loop switches the $8000 PRG bank and calls into
  it about every 200 instructions, switches CHR banks, arms the scanline IRQ at a line 20..220 that depends on
  the console's own history, and splits the scroll on the sprite-0 hit.
* ``smb_like_cart(seed)`` - NROM-128 that writes the RAM bytes the SMB reward reader reads (position, level,
  lives, score, dying, mode) from the pad, idling in a JMP-to-self loop with its logic in the NMI as SMB does,
  so rewards, deaths, level changes, game over and the idle fast-forward all run.
* ``dmc_cart(seed)`` - NROM-128 playing DMC samples (rate and loop changes, starts, stops, status polls).
* ``vblank_io_cart(seed)`` - NROM-128 whose NMI writes every PPU register in vblank (OAM through $2003/$2004 with
  the address wrapping, palette mirrors, a column with the increment of 32, register mirrors, an indexed store) and
  every fourth frame takes a nested NMI by turning NMI off and on while the vblank flag is up.
* ``poll_cart(seed)`` - NROM-128 with NMI off that polls instead: its main loop waits for vblank on $2002 bit 7,
  does the vblank work, waits for the sprite-0 flag to clear and then to be set (bit 6) and splits the scroll.
* ``fault_cart(nmis)`` - NROM-128 that hits an unofficial opcode after `nmis` frames (the emulator-fault end).
* ``mmc2_cart(seed)`` - MMC2 (mapper 9): 128 KB PRG in 8 KB banks, 128 KB CHR ROM, nametables and sprites rich in
  the latch tiles $FD/$FE, CHR bank and mirroring rewrites, CPU-driven latch flips through $2006/$2007.
* ``spec_cart(spec, seed)`` - NROM-128 that writes the RAM bytes a game's reward reader reads, from a spec of
  value lists and pad-driven walks, in its NMI (any of the twelve reward10 games).
* ``smb_ram15(seed, n_envs, steps)`` - per env-step the 15 RAM bytes the SMB reward reader reads (x position as a
  +-1..4 px random walk with 5% rollback jumps, world/level advancing with p 1e-3, lives lost with p 5e-4, BCD-like
  score digits), packed as ``rl10_smb_run`` takes them.

The RAM addresses the SMB reader reads (0x0E, 0x6D, 0x86, 0xB5, 0x75A-0x75F, 0x770, 0x772, 0x7DD-0x7E2) are never
written by the generated carts, so their reward stays 0 and no episode ends except by the stall clock.
"""
from __future__ import annotations

import numpy as np

# ------------------------------------------------------------------------------------------- assembler

_OPS = {
    'ADC': dict(imm=0x69, zp=0x65, zpx=0x75, abs=0x6D, abx=0x7D, aby=0x79, izx=0x61, izy=0x71),
    'AND': dict(imm=0x29, zp=0x25, zpx=0x35, abs=0x2D, abx=0x3D, aby=0x39, izx=0x21, izy=0x31),
    'ASL': dict(acc=0x0A, zp=0x06, zpx=0x16, abs=0x0E, abx=0x1E),
    'BCC': dict(rel=0x90), 'BCS': dict(rel=0xB0), 'BEQ': dict(rel=0xF0), 'BMI': dict(rel=0x30),
    'BNE': dict(rel=0xD0), 'BPL': dict(rel=0x10), 'BVC': dict(rel=0x50), 'BVS': dict(rel=0x70),
    'BIT': dict(zp=0x24, abs=0x2C),
    'BRK': dict(imp=0x00), 'CLC': dict(imp=0x18), 'CLD': dict(imp=0xD8), 'CLI': dict(imp=0x58), 'CLV': dict(imp=0xB8),
    'CMP': dict(imm=0xC9, zp=0xC5, zpx=0xD5, abs=0xCD, abx=0xDD, aby=0xD9, izx=0xC1, izy=0xD1),
    'CPX': dict(imm=0xE0, zp=0xE4, abs=0xEC), 'CPY': dict(imm=0xC0, zp=0xC4, abs=0xCC),
    'DEC': dict(zp=0xC6, zpx=0xD6, abs=0xCE, abx=0xDE), 'DEX': dict(imp=0xCA), 'DEY': dict(imp=0x88),
    'EOR': dict(imm=0x49, zp=0x45, zpx=0x55, abs=0x4D, abx=0x5D, aby=0x59, izx=0x41, izy=0x51),
    'INC': dict(zp=0xE6, zpx=0xF6, abs=0xEE, abx=0xFE), 'INX': dict(imp=0xE8), 'INY': dict(imp=0xC8),
    'JMP': dict(abs=0x4C, ind=0x6C), 'JSR': dict(abs=0x20),
    'LDA': dict(imm=0xA9, zp=0xA5, zpx=0xB5, abs=0xAD, abx=0xBD, aby=0xB9, izx=0xA1, izy=0xB1),
    'LDX': dict(imm=0xA2, zp=0xA6, zpy=0xB6, abs=0xAE, aby=0xBE),
    'LDY': dict(imm=0xA0, zp=0xA4, zpx=0xB4, abs=0xAC, abx=0xBC),
    'LSR': dict(acc=0x4A, zp=0x46, zpx=0x56, abs=0x4E, abx=0x5E), 'NOP': dict(imp=0xEA),
    'ORA': dict(imm=0x09, zp=0x05, zpx=0x15, abs=0x0D, abx=0x1D, aby=0x19, izx=0x01, izy=0x11),
    'PHA': dict(imp=0x48), 'PHP': dict(imp=0x08), 'PLA': dict(imp=0x68), 'PLP': dict(imp=0x28),
    'ROL': dict(acc=0x2A, zp=0x26, zpx=0x36, abs=0x2E, abx=0x3E),
    'ROR': dict(acc=0x6A, zp=0x66, zpx=0x76, abs=0x6E, abx=0x7E),
    'RTI': dict(imp=0x40), 'RTS': dict(imp=0x60),
    'SBC': dict(imm=0xE9, zp=0xE5, zpx=0xF5, abs=0xED, abx=0xFD, aby=0xF9, izx=0xE1, izy=0xF1),
    'SEC': dict(imp=0x38), 'SED': dict(imp=0xF8), 'SEI': dict(imp=0x78),
    'STA': dict(zp=0x85, zpx=0x95, abs=0x8D, abx=0x9D, aby=0x99, izx=0x81, izy=0x91),
    'STX': dict(zp=0x86, zpy=0x96, abs=0x8E), 'STY': dict(zp=0x84, zpx=0x94, abs=0x8C),
    'TAX': dict(imp=0xAA), 'TAY': dict(imp=0xA8), 'TSX': dict(imp=0xBA), 'TXA': dict(imp=0x8A),
    'TXS': dict(imp=0x9A), 'TYA': dict(imp=0x98),
}
_LEN = dict(imp=1, acc=1, imm=2, zp=2, zpx=2, zpy=2, izx=2, izy=2, rel=2, abs=3, abx=3, aby=3, ind=3)
OPCODES = {op: (mn, mode) for mn, modes in _OPS.items() for mode, op in modes.items()}  # the 151 official ones


class Asm:
    """Two-pass 6502 assembler: ``a.op('LDA', 'imm', 5)``, labels by name, ``a.byte(...)`` for data."""

    def __init__(self, origin: int):
        self.origin = origin
        self.items = []          # (kind, payload)
        self.labels = {}
        self.pc = origin

    def label(self, name):
        assert name not in self.labels, name
        self.labels[name] = self.pc
        return name

    def op(self, mn, mode='imp', arg=None):
        assert mode in _OPS[mn], (mn, mode)
        self.items.append(('op', (mn, mode, arg, self.pc)))
        self.pc += _LEN[mode]

    def byte(self, *vals):
        data = bytes(int(v) & 0xFF for v in vals)
        self.items.append(('data', data))
        self.pc += len(data)

    def data(self, buf):
        self.items.append(('data', bytes(buf)))
        self.pc += len(buf)

    def _val(self, arg):
        return self.labels[arg] if isinstance(arg, str) else int(arg)

    def assemble(self) -> bytes:
        out = bytearray()
        for kind, p in self.items:
            if kind == 'data':
                out += p
                continue
            mn, mode, arg, pc = p
            out.append(_OPS[mn][mode])
            if mode == 'rel':
                d = self._val(arg) - (pc + 2)
                assert -128 <= d <= 127, f'branch out of range at {pc:04x}'
                out.append(d & 0xFF)
            elif _LEN[mode] == 2:
                v = self._val(arg)
                assert 0 <= v <= 0xFF, (mn, mode, v)
                out.append(v)
            elif _LEN[mode] == 3:
                v = self._val(arg)
                out += bytes((v & 0xFF, (v >> 8) & 0xFF))
        return bytes(out)


def ines(prg: bytes, chr_: bytes, mapper: int, vertical: bool = True, submapper: int = None) -> bytes:
    """iNES image; with a submapper, an NES 2.0 header (byte 7 bits 2-3 = 2, submapper in byte 8 bits 4-7)."""
    assert len(prg) % 16384 == 0 and len(chr_) % 8192 == 0
    h = bytearray(b'NES\x1a')
    h += bytes((len(prg) // 16384, len(chr_) // 8192, ((mapper & 15) << 4) | (1 if vertical else 0),
                (mapper & 0xF0) | (0x08 if submapper is not None else 0)))
    h += bytes(8)
    if submapper is not None:
        h[8] = (submapper & 15) << 4
    return bytes(h) + prg + chr_


# ------------------------------------------------------------------------------------- code builders

# zero-page / RAM map of the generated programs (none of the SMB reader's addresses)
PAD, CTRL_SHADOW, PX, PY, ACNT, TSEL, BACC = 0x10, 0x11, 0x20, 0x21, 0x22, 0x23, 0x24
CNT_LO, CNT_HI, NTP_LO, NTP_HI, FRAMES, NMIFLAG, BANK, IRQLINE = 0x30, 0x31, 0x32, 0x33, 0x40, 0x41, 0x42, 0x43
SCRATCH_ZP = list(range(0x50, 0x6C))      # stays below 0x6D
WORK_PAGE = 0x0300                        # 256 B work area
OAM_PAGE = 0x0200


def _filler(a: Asm, rng: np.random.Generator, nblocks: int, tag: str, table: str, with_prg_ram=False):
    """Seeded blocks of 6502 work on RAM counters: arithmetic, shifts, table lookups, short loops and
    data- and pad-dependent branches (so consoles with different pads take different paths)."""
    zp = lambda: int(rng.choice(SCRATCH_ZP))  # noqa: E731
    for i in range(nblocks):
        k = int(rng.integers(0, 9 if with_prg_ram else 8))
        lab = f'{tag}_{i}'
        if k == 0:
            a.op('LDA', 'zp', zp()); a.op('CLC'); a.op('ADC', 'zp', zp()); a.op('STA', 'zp', zp())
        elif k == 1:
            a.op('LDA', 'zp', zp()); a.op('ASL', 'acc'); a.op('EOR', 'imm', int(rng.integers(256)))
            a.op('STA', 'zp', zp())
        elif k == 2:
            a.op('LDX', 'zp', zp()); a.op('LDA', 'abx', table); a.op('STA', 'abx', WORK_PAGE)
        elif k == 3:
            a.op('LDY', 'imm', int(rng.integers(3, 12)))
            a.label(lab + 'l')
            a.op('LDA', 'aby', WORK_PAGE); a.op('ADC', 'imm', int(rng.integers(256))); a.op('STA', 'aby', WORK_PAGE)
            a.op('DEY'); a.op('BNE', 'rel', lab + 'l')
        elif k == 4:
            a.op('LDA', 'zp', zp()); a.op('AND', 'imm', int(1 << rng.integers(8))); a.op('BEQ', 'rel', lab)
            a.op('INC', 'zp', zp()); a.op('LDA', 'zp', CNT_LO); a.op('STA', 'zp', zp())
            a.label(lab)
        elif k == 5:
            a.op('LDA', 'zp', PAD); a.op('AND', 'imm', int(1 << rng.integers(8))); a.op('BNE', 'rel', lab)
            a.op('LDA', 'zp', zp()); a.op('ROR', 'acc'); a.op('STA', 'zp', zp()); a.op('INC', 'abs', WORK_PAGE + int(rng.integers(256)))
            a.label(lab)
        elif k == 6:
            a.op('LDA', 'zp', zp()); a.op('SEC'); a.op('SBC', 'zp', zp()); a.op('BCS', 'rel', lab)
            a.op('EOR', 'imm', 0xFF); a.op('LSR', 'acc')
            a.label(lab)
            a.op('STA', 'zp', zp())
        elif k == 7:
            a.op('LDA', 'zp', PX); a.op('CMP', 'zp', PY); a.op('BCC', 'rel', lab)
            a.op('LDA', 'zp', ACNT); a.op('AND', 'imm', 0x0F); a.op('TAX')
            a.op('INC', 'zpx', 0x50); a.op('LDA', 'zpx', 0x50); a.op('STA', 'zp', zp())
            a.label(lab)
        else:
            a.op('LDX', 'zp', zp()); a.op('LDA', 'abx', 0x6000); a.op('ADC', 'zp', zp()); a.op('STA', 'abx', 0x6000)


def _read_pad(a: Asm, tag: str):
    a.op('LDA', 'imm', 1); a.op('STA', 'abs', 0x4016); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x4016)
    a.op('LDX', 'imm', 8)
    a.label(tag + 'rd')
    a.op('LDA', 'abs', 0x4016); a.op('LSR', 'acc'); a.op('ROR', 'zp', PAD); a.op('DEX'); a.op('BNE', 'rel', tag + 'rd')


def _pad_moves(a: Asm, table: str):
    for bit, op, var, lab in ((0x80, 'INC', PX, 'nr'), (0x40, 'DEC', PX, 'nl'), (0x20, 'INC', PY, 'nd'),
                              (0x10, 'DEC', PY, 'nu')):
        a.op('LDA', 'zp', PAD); a.op('AND', 'imm', bit); a.op('BEQ', 'rel', 'mv_' + lab); a.op(op, 'zp', var)
        a.label('mv_' + lab)
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x01); a.op('BEQ', 'rel', 'mv_na')
    a.op('INC', 'zp', ACNT); a.op('LDA', 'zp', ACNT); a.op('AND', 'imm', 0x0F); a.op('TAX'); a.op('LDA', 'abx', table)
    a.op('STA', 'zp', TSEL)
    a.label('mv_na')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x02); a.op('BEQ', 'rel', 'mv_nb')
    a.op('LDA', 'zp', BACC); a.op('CLC'); a.op('ADC', 'zp', PX); a.op('STA', 'zp', BACC)
    a.label('mv_nb')
    a.op('INC', 'zp', CNT_LO); a.op('BNE', 'rel', 'mv_c1'); a.op('INC', 'zp', CNT_HI)
    a.label('mv_c1')


def _reset_common(a: Asm, ctrl: int, tables: dict):
    a.op('SEI'); a.op('CLD'); a.op('LDX', 'imm', 0xFF); a.op('TXS')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2000); a.op('STA', 'abs', 0x2001)
    for k in range(2):
        a.label(f'vw{k}'); a.op('BIT', 'abs', 0x2002); a.op('BPL', 'rel', f'vw{k}')
    a.op('LDA', 'imm', 0); a.op('TAX')
    a.label('clr')
    for page in range(8):
        a.op('STA', 'abx', page * 256)
    a.op('INX'); a.op('BNE', 'rel', 'clr')
    # palette
    a.op('LDA', 'abs', 0x2002)
    a.op('LDA', 'imm', 0x3F); a.op('STA', 'abs', 0x2006); a.op('LDA', 'imm', 0x00); a.op('STA', 'abs', 0x2006)
    a.op('LDX', 'imm', 0)
    a.label('pal'); a.op('LDA', 'abx', tables['pal']); a.op('STA', 'abs', 0x2007); a.op('INX'); a.op('CPX', 'imm', 32)
    a.op('BNE', 'rel', 'pal')
    # both nametables: the 256-byte table, offset by the page number
    a.op('LDA', 'imm', 0x20); a.op('STA', 'abs', 0x2006); a.op('LDA', 'imm', 0x00); a.op('STA', 'abs', 0x2006)
    a.op('LDY', 'imm', 8); a.op('LDX', 'imm', 0)
    a.label('ntl'); a.op('TYA'); a.op('CLC'); a.op('ADC', 'abx', tables['nt']); a.op('STA', 'abs', 0x2007); a.op('INX')
    a.op('BNE', 'rel', 'ntl'); a.op('DEY'); a.op('BNE', 'rel', 'ntl')
    # OAM buffer
    a.op('LDX', 'imm', 0)
    a.label('oam'); a.op('LDA', 'abx', tables['oam']); a.op('STA', 'abx', OAM_PAGE); a.op('INX'); a.op('BNE', 'rel', 'oam')
    a.op('LDA', 'imm', 0x80); a.op('STA', 'zp', PX); a.op('LDA', 'imm', 0x70); a.op('STA', 'zp', PY)
    a.op('LDA', 'imm', 0x20); a.op('STA', 'zp', NTP_HI)
    a.op('LDA', 'imm', ctrl); a.op('STA', 'zp', CTRL_SHADOW); a.op('STA', 'abs', 0x2000)
    a.op('LDA', 'imm', 0x1E); a.op('STA', 'abs', 0x2001)


def _nmi_common(a: Asm):
    a.op('PHA'); a.op('TXA'); a.op('PHA'); a.op('TYA'); a.op('PHA')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2003); a.op('LDA', 'imm', OAM_PAGE >> 8); a.op('STA', 'abs', 0x4014)
    a.op('LDA', 'zp', PY); a.op('STA', 'abs', OAM_PAGE + 4); a.op('LDA', 'zp', PX); a.op('STA', 'abs', OAM_PAGE + 7)
    a.op('LDA', 'abs', 0x2002)
    a.op('LDA', 'zp', NTP_HI); a.op('STA', 'abs', 0x2006); a.op('LDA', 'zp', NTP_LO); a.op('STA', 'abs', 0x2006)
    for v in (CNT_LO, CNT_HI, ACNT, PAD):
        a.op('LDA', 'zp', v); a.op('STA', 'abs', 0x2007)
    a.op('LDA', 'zp', NTP_LO); a.op('CLC'); a.op('ADC', 'imm', 4); a.op('STA', 'zp', NTP_LO)
    a.op('LDA', 'zp', NTP_HI); a.op('ADC', 'imm', 0); a.op('AND', 'imm', 0x03); a.op('ORA', 'imm', 0x20)
    a.op('STA', 'zp', NTP_HI)
    a.op('LDA', 'zp', PX); a.op('STA', 'abs', 0x2005); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2005)
    a.op('LDA', 'zp', CTRL_SHADOW); a.op('STA', 'abs', 0x2000)
    a.op('INC', 'zp', FRAMES); a.op('LDA', 'imm', 1); a.op('STA', 'zp', NMIFLAG)


def _nmi_end(a: Asm):
    a.op('PLA'); a.op('TAY'); a.op('PLA'); a.op('TAX'); a.op('PLA'); a.op('RTI')


def _tables(rng):
    pal = rng.integers(0, 64, 32)
    nt = rng.integers(0, 256, 256)
    oam = np.empty(256, np.int64)
    oam[0::4] = rng.integers(0, 0xF0, 64)
    oam[1::4] = rng.integers(0, 256, 64)
    oam[2::4] = rng.integers(0, 256, 64) & 0xE3
    oam[3::4] = rng.integers(0, 256, 64)
    mix = rng.integers(0, 256, 256)
    return pal, nt, oam, mix


def nrom_cart(seed: int = 0, blocks: int = 24) -> bytes:
    """NROM-128 cartridge: 16 KB PRG (code at $C000, mirrored at $8000) + 8 KB random CHR."""
    rng = np.random.default_rng([0x4E524F4D, seed])
    pal, nt, oam, mix = _tables(rng)
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    _filler(a, rng, blocks, 'f', 't_mix')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


# (ctrl, mask) of the modes cart's frames, FRAMES & 7: 8x8 and 8x16 sprites from either pattern table, sprites or
# the background off, the left column clipped for either or both, greyscale and emphasis.
MODES = ((0x90, 0x1E), (0xB0, 0x1E), (0x90, 0x0E), (0xB0, 0x16), (0x98, 0x18), (0xB8, 0x1A), (0x90, 0x1F),
         (0xB0, 0x3E))


def modes_cart(seed: int = 0, blocks: int = 12) -> bytes:
    """NROM-128 cartridge like nrom_cart whose NMI also sets the next frame's PPU mode from MODES by its frame counter
    (both writes inside vblank, so every visible line of a frame is drawn in one mode)."""
    rng = np.random.default_rng([0x4D4F4445, seed])
    pal, nt, oam, mix = _tables(rng)
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    _filler(a, rng, blocks, 'f', 't_mix')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 7); a.op('TAX')
    a.op('LDA', 'abx', 't_ctrl'); a.op('STA', 'abs', 0x2000); a.op('LDA', 'abx', 't_mask'); a.op('STA', 'abs', 0x2001)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix), ('t_ctrl', [c for c, _ in MODES]),
                    ('t_mask', [m for _, m in MODES])):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


NMI_DEPTH, NESTED = 0x26, 0x27           # the vblank I/O cart's NMI nesting flag and its count of nested NMIs


def vblank_io_cart(seed: int = 0, blocks: int = 12) -> bytes:
    """NROM-128 cartridge like nrom_cart whose NMI, between vblank and the pre-render line, uses every PPU register
    write there is: every fourth frame it turns NMI off and on again before reading $2002, so the still-raised vblank
    flag takes a second (nested) NMI, which counts itself in NESTED and returns; then the OAM DMA and an OAM patch
    through $2003/$2004 (the entry of sprite (FRAMES & 15) + 2, and every eighth frame four bytes from $FE on, which
    wrap into sprite 0), one palette entry (FRAMES & 31, the $3F10 mirrors included), six nametable bytes down a
    column with the increment of 32 through the $2007 mirror $2FFF, one byte by an indexed store (STA $2000,X), a
    buffered $2007 read, the four counter bytes and the scroll through the $2005 mirror $3FFD, and the mask through
    $3FF9."""
    rng = np.random.default_rng([0x56494F00, seed])
    pal, nt, oam, mix = _tables(rng)
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    _filler(a, rng, blocks, 'f', 't_mix')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    a.op('PHA'); a.op('TXA'); a.op('PHA'); a.op('TYA'); a.op('PHA')
    a.op('LDA', 'zp', NMI_DEPTH); a.op('BEQ', 'rel', 'vio_first')
    a.op('INC', 'zp', NESTED); a.op('JMP', 'abs', 'vio_out')
    a.label('vio_first')
    a.op('INC', 'zp', NMI_DEPTH)
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 3); a.op('BNE', 'rel', 'vio_dma')
    a.op('LDA', 'imm', 0x10); a.op('STA', 'abs', 0x2000); a.op('LDA', 'imm', 0x90); a.op('STA', 'abs', 0x2000)
    a.label('vio_dma')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2003); a.op('LDA', 'imm', OAM_PAGE >> 8); a.op('STA', 'abs', 0x4014)
    # sprite (FRAMES & 15) + 2: y, tile, attributes, x
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 15); a.op('CLC'); a.op('ADC', 'imm', 2); a.op('ASL', 'acc')
    a.op('ASL', 'acc'); a.op('STA', 'abs', 0x2003)
    a.op('LDA', 'zp', PY); a.op('CLC'); a.op('ADC', 'imm', 16); a.op('STA', 'abs', 0x2004)
    a.op('LDA', 'zp', CNT_LO); a.op('STA', 'abs', 0x2004)
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 0xE3); a.op('STA', 'abs', 0x2004)
    a.op('LDA', 'zp', PX); a.op('EOR', 'imm', 0x55); a.op('STA', 'abs', 0x2004)
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 7); a.op('BNE', 'rel', 'vio_nowrap')
    a.op('LDA', 'imm', 0xFE); a.op('STA', 'abs', 0x2003)
    for v in (0x21, 0x40, 0x30, 0x00):    # sprite 63's attributes and x, then sprite 0's y and tile
        a.op('LDA', 'imm', v); a.op('EOR', 'zp', FRAMES); a.op('STA', 'abs', 0x2004)
    a.label('vio_nowrap')
    a.op('LDA', 'zp', PY); a.op('STA', 'abs', OAM_PAGE + 4); a.op('LDA', 'zp', PX); a.op('STA', 'abs', OAM_PAGE + 7)
    a.op('LDA', 'abs', 0x2002)
    # palette entry FRAMES & 31
    a.op('LDA', 'imm', 0x3F); a.op('STA', 'abs', 0x2006); a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 0x1F)
    a.op('STA', 'abs', 0x2006); a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('STA', 'abs', 0x2007)
    # a column: nametable 1 or 3 (FRAMES bit 5; the counter bytes below go to nametable 0), column FRAMES & 31,
    # 6 bytes with the increment of 32
    a.op('LDA', 'imm', 0x94); a.op('STA', 'abs', 0x2000)
    a.op('LDA', 'zp', FRAMES); a.op('LSR', 'acc'); a.op('LSR', 'acc'); a.op('AND', 'imm', 0x08); a.op('ORA', 'imm', 0x24)
    a.op('STA', 'abs', 0x2006); a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 0x1F); a.op('STA', 'abs', 0x2006)
    a.op('LDX', 'imm', 6)
    a.label('vio_col')
    a.op('TXA'); a.op('EOR', 'zp', FRAMES); a.op('STA', 'abs', 0x2FFF); a.op('DEX'); a.op('BNE', 'rel', 'vio_col')
    a.op('LDA', 'imm', 0x90); a.op('STA', 'abs', 0x2000)
    a.op('LDX', 'imm', 7); a.op('LDA', 'zp', PAD); a.op('STA', 'abx', 0x2000)
    a.op('LDA', 'abs', 0x2007)
    a.op('LDA', 'zp', NTP_HI); a.op('STA', 'abs', 0x2006); a.op('LDA', 'zp', NTP_LO); a.op('STA', 'abs', 0x2006)
    for v in (CNT_LO, CNT_HI, ACNT, PAD):
        a.op('LDA', 'zp', v); a.op('STA', 'abs', 0x2007)
    a.op('LDA', 'zp', NTP_LO); a.op('CLC'); a.op('ADC', 'imm', 4); a.op('STA', 'zp', NTP_LO)
    a.op('LDA', 'zp', NTP_HI); a.op('ADC', 'imm', 0); a.op('AND', 'imm', 0x03); a.op('ORA', 'imm', 0x20)
    a.op('STA', 'zp', NTP_HI)
    a.op('LDA', 'zp', PX); a.op('STA', 'abs', 0x3FFD); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x3FFD)
    a.op('LDA', 'zp', CTRL_SHADOW); a.op('STA', 'abs', 0x2000); a.op('LDA', 'imm', 0x1E); a.op('STA', 'abs', 0x3FF9)
    a.op('INC', 'zp', FRAMES); a.op('LDA', 'imm', 1); a.op('STA', 'zp', NMIFLAG)
    a.op('LDA', 'imm', 0); a.op('STA', 'zp', NMI_DEPTH)
    a.label('vio_out')
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


def poll_cart(seed: int = 0, blocks: int = 12, bmi: bool = False) -> bytes:
    """NROM-128 cartridge with NMI off: every frame of its main loop waits for vblank with BIT $2002 / BPL, writes the
    OAM (DMA), the sprite's position, four nametable bytes and the scroll, waits for the sprite-0 flag to clear (BIT /
    BVS) and to be set again (BIT / BVC), splits the scroll there, then reads the pad and runs the filler blocks.
    Sprite 0 sits over the random background at (x, 96), so its hit comes on every frame.

    bmi: the loop then also spins for 10 + (pad & 7) times 1,284 cycles, which ends before, inside or after vblank
    depending on the pad, and waits on BIT $2002 / BMI back to itself: inside vblank that read sees the flag set,
    clears it and branches, and the next read falls through."""
    rng = np.random.default_rng([0x504F4C4C, seed])
    pal, nt, oam, mix = _tables(rng)
    oam[0], oam[1], oam[2], oam[3] = 95, int(rng.integers(1, 256)), 0, int(rng.integers(16, 200))
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x10, tables)
    a.label('main')
    a.label('p_vb'); a.op('BIT', 'abs', 0x2002); a.op('BPL', 'rel', 'p_vb')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2003); a.op('LDA', 'imm', OAM_PAGE >> 8); a.op('STA', 'abs', 0x4014)
    a.op('LDA', 'zp', PY); a.op('STA', 'abs', OAM_PAGE + 4); a.op('LDA', 'zp', PX); a.op('STA', 'abs', OAM_PAGE + 7)
    a.op('LDA', 'abs', 0x2002)
    a.op('LDA', 'zp', NTP_HI); a.op('STA', 'abs', 0x2006); a.op('LDA', 'zp', NTP_LO); a.op('STA', 'abs', 0x2006)
    for v in (CNT_LO, CNT_HI, ACNT, PAD):
        a.op('LDA', 'zp', v); a.op('STA', 'abs', 0x2007)
    a.op('LDA', 'zp', NTP_LO); a.op('CLC'); a.op('ADC', 'imm', 4); a.op('STA', 'zp', NTP_LO)
    a.op('LDA', 'zp', NTP_HI); a.op('ADC', 'imm', 0); a.op('AND', 'imm', 0x03); a.op('ORA', 'imm', 0x20)
    a.op('STA', 'zp', NTP_HI)
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2005); a.op('STA', 'abs', 0x2005)
    a.op('LDA', 'zp', CTRL_SHADOW); a.op('STA', 'abs', 0x2000)
    a.label('p_s0c'); a.op('BIT', 'abs', 0x2002); a.op('BVS', 'rel', 'p_s0c')
    a.label('p_s0h'); a.op('BIT', 'abs', 0x2002); a.op('BVC', 'rel', 'p_s0h')
    a.op('LDA', 'zp', PX); a.op('STA', 'abs', 0x2005); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2005)
    a.op('INC', 'zp', FRAMES)
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    _filler(a, rng, blocks, 'f', 't_mix')
    if bmi:
        a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 7); a.op('CLC'); a.op('ADC', 'imm', 10); a.op('TAY')
        a.label('p_dy'); a.op('LDX', 'imm', 0)
        a.label('p_dx'); a.op('DEX'); a.op('BNE', 'rel', 'p_dx')
        a.op('DEY'); a.op('BNE', 'rel', 'p_dy')
        a.label('p_bm'); a.op('BIT', 'abs', 0x2002); a.op('BMI', 'rel', 'p_bm')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    a.op('RTI')
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


DMC_CNT = 0x25                            # the DMC cart's count of status polls that saw a sample playing


def dmc_cart(seed: int = 0, blocks: int = 16) -> bytes:
    """NROM-128 cartridge that plays DMC samples: every pass of its main loop writes a rate ($4010 bits 0-3, changed
    while a sample plays) and the loop flag (bit 6) from its counters, a length ($4013) from the pad, starts a sample
    ($4015 = $10) every 32 passes and stops it ($4015 = 0) every 64, and polls $4015 bit 4 (bytes left) up to 8 times.
    Each sample byte fetched steals 4 CPU cycles, so the console's timing, and with it every later frame, depends on
    the channel."""
    rng = np.random.default_rng([0x444D4320, seed])
    pal, nt, oam, mix = _tables(rng)
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 0x4F); a.op('STA', 'abs', 0x4010)
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x07); a.op('STA', 'abs', 0x4013)
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x1F); a.op('BNE', 'rel', 'd_nostart')
    a.op('LDA', 'imm', 0x10); a.op('STA', 'abs', 0x4015)
    a.label('d_nostart')
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x3F); a.op('CMP', 'imm', 0x30); a.op('BNE', 'rel', 'd_nostop')
    a.op('LDA', 'imm', 0x00); a.op('STA', 'abs', 0x4015)
    a.label('d_nostop')
    a.op('LDX', 'imm', 8)
    a.label('d_poll'); a.op('LDA', 'abs', 0x4015); a.op('AND', 'imm', 0x10); a.op('BEQ', 'rel', 'd_done')
    a.op('INC', 'zp', DMC_CNT); a.op('DEX'); a.op('BNE', 'rel', 'd_poll')
    a.label('d_done')
    _filler(a, rng, blocks, 'f', 't_mix')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


def fault_cart(nmis: int = 3) -> bytes:
    """NROM-128 cartridge that runs into an unofficial opcode ($02) once its NMI has counted `nmis` frames: an
    emulator fault, which ends the episode (end reason 5, reward 0; rl/csrc/rlenv_core.cuh:273-301)."""
    a = Asm(0xC000)
    a.label('reset')
    a.op('SEI'); a.op('LDA', 'imm', 0); a.op('STA', 'zp', 0x10); a.op('LDA', 'imm', 0x80); a.op('STA', 'abs', 0x2000)
    a.op('LDA', 'imm', 0x1E); a.op('STA', 'abs', 0x2001)
    a.label('loop')
    a.op('LDA', 'zp', 0x10); a.op('CMP', 'imm', nmis); a.op('BCC', 'rel', 'loop')
    a.byte(0x02)
    a.label('nmi')
    a.op('INC', 'zp', 0x10); a.op('RTI')
    code = a.assemble()
    prg = bytearray(16384)
    prg[:len(code)] = code
    prg[0x3FFA:0x4000] = bytes((a.labels['nmi'] & 0xFF, a.labels['nmi'] >> 8, 0, 0xC0, 0, 0xC0))
    return ines(bytes(prg), bytes(range(256)) * 32, 0)


def cnrom_cart(seed: int = 0, blocks: int = 24, conflicts: bool = False) -> bytes:
    """CNROM cartridge: 32 KB PRG at $8000, 32 KB CHR in four 8 KB banks. The NMI selects bank FRAMES & 3 and the
    main loop selects one mid-frame from the counter and the pad, both by storing the bank number over a ROM byte
    that holds it (no bus conflict). With conflicts, the header declares AND-type bus conflicts (NES 2.0 submapper 2)
    and the main loop also stores $FF over a byte holding 2 when pad bit 6 is set: bank 2 there, bank 3 without
    conflicts."""
    rng = np.random.default_rng([0x434E524D, seed])
    pal, nt, oam, mix = _tables(rng)
    a = Asm(0x8000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    _filler(a, rng, blocks // 2, 'f', 't_mix')
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 3); a.op('TAX')
    a.op('STA', 'abx', 't_bank')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x40); a.op('BEQ', 'rel', 'no_cf')
    a.op('LDA', 'imm', 0xFF); a.op('STA', 'abs', 't_two')
    a.label('no_cf')
    _filler(a, rng, blocks - blocks // 2, 'g', 't_mix')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 3); a.op('TAX'); a.op('STA', 'abx', 't_bank')
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    a.label('t_bank')
    a.data(bytes((0, 1, 2, 3)))
    a.label('t_two')
    a.data(bytes((2,)))
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x7FFA, len(code)
    prg = bytearray(32768)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x7FFA:0x8000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 32768, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 3, vertical=True, submapper=2 if conflicts else None)


def uxrom_cart(seed: int = 0, blocks: int = 16, sub_blocks: int = 16, conflicts: bool = False) -> bytes:
    """UxROM cartridge: 128 KB PRG in 16 KB banks (banks 0-6 hold seeded subroutines at $8000, bank 7 is fixed at
    $C000), 8 KB random CHR. The main loop selects a bank from the counter and the pad by storing the bank number
    over a ROM byte that holds it, and calls the subroutine there. With conflicts, the header declares AND-type bus
    conflicts (NES 2.0 submapper 2) and the main loop also stores $FF over a byte holding 5 when pad bit 6 is set:
    bank 5 there, bank 7 without conflicts."""
    rng = np.random.default_rng([0x55584F4D, seed])
    pal, nt, oam, mix = _tables(rng)
    banks = []
    for b in range(7):
        s = Asm(0x8000)
        _filler(s, rng, sub_blocks, f'b{b}', 0xBF00)
        s.op('RTS')
        body = s.assemble()
        page = bytearray(16384)
        page[:len(body)] = body
        page[0x3F00:0x4000] = rng.integers(0, 256, 256, dtype=np.uint8).tobytes()   # table at $BF00
        banks.append(bytes(page))
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.op('RTS')                                          # bank 7 at $8000 (the $FF store): the call returns
    a.label('reset')
    _reset_common(a, 0x90, tables)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 7); a.op('CMP', 'imm', 7)
    a.op('BCC', 'rel', 'bk_ok'); a.op('LDA', 'imm', 2)
    a.label('bk_ok')
    a.op('TAX'); a.op('STA', 'abx', 't_bank')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x40); a.op('BEQ', 'rel', 'no_cf')
    a.op('LDA', 'imm', 0xFF); a.op('STA', 'abs', 't_five')
    a.label('no_cf')
    a.op('JSR', 'abs', 0x8000)
    _filler(a, rng, blocks, 'f', 't_mix')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    a.label('t_bank')
    a.data(bytes(range(8)))
    a.label('t_five')
    a.data(bytes((5,)))
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    fixed = bytearray(16384)
    fixed[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    fixed[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(b''.join(banks) + bytes(fixed), chr_, 2, vertical=False, submapper=2 if conflicts else None)


def mmc3_cart(seed: int = 0, blocks: int = 16, sub_blocks: int = 20) -> bytes:
    """MMC3 cartridge: 256 KB PRG (32 x 8 KB; banks 0-29 hold seeded subroutines at $8000, bank 30 at $C000 and
    bank 31 at $E000 are fixed), 128 KB random CHR, scanline IRQ split, sprite-0 split, PRG RAM use."""
    rng = np.random.default_rng([0x4D4D4333, seed])
    pal, nt, oam, mix = _tables(rng)
    oam[0:4] = (24, int(rng.integers(256)), 0x00, 40)        # sprite 0 over the playfield near the top
    banks = []
    for b in range(30):   # switchable: a subroutine at $8000
        s = Asm(0x8000)
        _filler(s, rng, sub_blocks, f's{b}', 0x9F00, with_prg_ram=True)
        s.op('RTS')
        body = s.assemble()
        page = bytearray(8192)
        page[:len(body)] = body
        page[0x1F00:0x2000] = rng.integers(0, 256, 256, dtype=np.uint8).tobytes()   # table at $9F00
        banks.append(bytes(page))
    # fixed banks: $C000-$DFFF tables + helpers, $E000-$FFFF code and vectors
    a = Asm(0xC000)
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    a.label('chrsw')          # CHR banks: R0/R1 (background 2 KB) and R2..R5 (sprites) from the counters
    for reg, var, mask in ((0, CNT_LO, 0x7E), (1, ACNT, 0x7E), (2, FRAMES, 0x7F), (5, BACC, 0x7F)):
        a.op('LDA', 'imm', reg); a.op('STA', 'abs', 0x8000); a.op('LDA', 'zp', var); a.op('AND', 'imm', mask)
        a.op('STA', 'abs', 0x8001)
    a.op('RTS')
    code_c = a.assemble()
    assert len(code_c) <= 0x2000
    a = Asm(0xE000)
    a.labels.update({k: v for k, v in (('t_pal', 0xC000), ('t_nt', 0xC020), ('t_oam', 0xC120), ('t_mix', 0xC220),
                                       ('chrsw', 0xC320))})
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    a.op('LDA', 'imm', 0x40); a.op('STA', 'abs', 0x4017)            # (APU frame IRQ off; ignored here)
    a.op('LDA', 'imm', 0x80); a.op('STA', 'abs', 0xA001)            # PRG RAM on
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0xA000)                # vertical mirroring
    _reset_common(a, 0x88, tables)                                   # NMI on, sprites at $1000, BG at $0000
    a.op('LDA', 'imm', 100); a.op('STA', 'zp', IRQLINE)
    a.op('CLI')
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    # sprite-0 split once per frame, after the NMI (bounded wait)
    a.op('LDA', 'zp', NMIFLAG); a.op('BEQ', 'rel', 's0_skip')
    a.op('LDA', 'imm', 0); a.op('STA', 'zp', NMIFLAG)
    a.op('LDX', 'imm', 0)
    a.label('s0_w'); a.op('BIT', 'abs', 0x2002); a.op('BVS', 'rel', 's0_hit'); a.op('DEX'); a.op('BNE', 'rel', 's0_w')
    a.label('s0_hit')
    a.op('LDA', 'zp', BACC); a.op('STA', 'abs', 0x2005); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2005)
    a.label('s0_skip')
    # switch the $8000 bank (R6) and call the subroutine there
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 0x1F); a.op('CMP', 'imm', 30)
    a.op('BCC', 'rel', 'bk_ok'); a.op('SBC', 'imm', 30)
    a.label('bk_ok')
    a.op('STA', 'zp', BANK)
    a.op('LDA', 'imm', 6); a.op('STA', 'abs', 0x8000); a.op('LDA', 'zp', BANK); a.op('STA', 'abs', 0x8001)
    a.op('JSR', 'abs', 0x8000)
    _filler(a, rng, blocks, 'f', 't_mix', with_prg_ram=True)
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x07); a.op('BNE', 'rel', 'no_chr'); a.op('JSR', 'abs', 'chrsw')
    a.label('no_chr')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    # next frame's IRQ line: 20 + (frames * 7 + pad) mod 200
    a.op('LDA', 'zp', FRAMES); a.op('ASL', 'acc'); a.op('ASL', 'acc'); a.op('ASL', 'acc'); a.op('SEC')
    a.op('SBC', 'zp', FRAMES); a.op('CLC'); a.op('ADC', 'zp', PAD)
    a.label('irq_mod'); a.op('CMP', 'imm', 200); a.op('BCC', 'rel', 'irq_ok'); a.op('SBC', 'imm', 200)
    a.op('JMP', 'abs', 'irq_mod')
    a.label('irq_ok')
    a.op('CLC'); a.op('ADC', 'imm', 20); a.op('STA', 'zp', IRQLINE)
    a.op('STA', 'abs', 0xC000); a.op('STA', 'abs', 0xC001); a.op('STA', 'abs', 0xE001)
    _nmi_end(a)
    a.label('irq')
    a.op('PHA')
    a.op('STA', 'abs', 0xE000)                                        # acknowledge + disable
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x8000); a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 0x7E)
    a.op('STA', 'abs', 0x8001)                                        # background bank split
    a.op('LDA', 'zp', PY); a.op('STA', 'abs', 0x2005); a.op('STA', 'abs', 0x2005)
    a.op('PLA'); a.op('RTI')
    code_e = a.assemble()
    assert a.labels['t_mix'] == 0xC220 and len(code_e) <= 0x1FFA, len(code_e)
    fixed_c = bytearray(8192)
    fixed_c[:len(code_c)] = code_c
    fixed_e = bytearray(8192)
    fixed_e[:len(code_e)] = code_e
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    fixed_e[0x1FFA:0x2000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    prg = b''.join(banks) + bytes(fixed_c) + bytes(fixed_e)
    chr_ = rng.integers(0, 256, 128 * 1024, dtype=np.uint8).tobytes()
    return ines(prg, chr_, 4, vertical=True)


MMC1_CTRL = 0x46                          # the MMC1 cart's shadow of its control register


def _mmc1_write(a: Asm, addr: int):
    """MMC1 serial port: the 5 low bits of A, least significant first (A is shifted out)."""
    for _ in range(4):
        a.op('STA', 'abs', addr); a.op('LSR', 'acc')
    a.op('STA', 'abs', addr)


def mmc1_cart(seed: int = 0, blocks: int = 16, sub_blocks: int = 16) -> bytes:
    """MMC1 cartridge in the layout of the MMC1 games of the set: 128 KB PRG in 16 KB banks (mode 3: banks 0-6
    switched in at $8000, bank 7 fixed at $C000), 8 KB CHR RAM filled by the program, PRG RAM at $6000.
    The main loop switches the $8000 bank through the serial port and calls the subroutine there, works on PRG RAM,
    and flips the mirroring now and then; the NMI rewrites one CHR RAM tile per frame (an animated tile)."""
    rng = np.random.default_rng([0x4D4D4331, seed])
    pal, nt, oam, mix = _tables(rng)
    banks = []
    for b in range(7):   # switchable: a subroutine at $8000
        s = Asm(0x8000)
        _filler(s, rng, sub_blocks, f'b{b}', 0xBF00, with_prg_ram=True)
        s.op('RTS')
        body = s.assemble()
        page = bytearray(16384)
        page[:len(body)] = body
        page[0x3F00:0x4000] = rng.integers(0, 256, 256, dtype=np.uint8).tobytes()   # table at $BF00
        banks.append(bytes(page))
    tiles = rng.integers(0, 256, 4096, dtype=np.uint8)
    a = Asm(0xE000)
    a.labels.update({k: v for k, v in (('t_pal', 0xC000), ('t_nt', 0xC020), ('t_oam', 0xC120), ('t_mix', 0xC220),
                                       ('t_tiles', 0xD000))})
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    a.op('SEI'); a.op('LDA', 'imm', 0x80); a.op('STA', 'abs', 0x8000)   # serial port reset: PRG mode 3
    a.op('LDA', 'imm', 0x0E); _mmc1_write(a, 0x8000)                      # vertical, PRG mode 3, CHR 8 KB
    a.op('LDA', 'imm', 0); _mmc1_write(a, 0xE000)                         # bank 0, PRG RAM on
    _reset_common(a, 0x80, tables)                                        # NMI on, BG and sprites at $0000
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2000); a.op('STA', 'abs', 0x2001)   # NMI and rendering off: upload
    a.op('LDA', 'abs', 0x2002); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2006); a.op('STA', 'abs', 0x2006)
    a.op('LDY', 'imm', 0)
    for half in range(2):                                                 # 2 x 4 KB of tiles
        for page in range(16):
            a.label(f'up{half}_{page}')
            a.op('LDA', 'aby', 0xD000 + page * 256)
            if half:
                a.op('EOR', 'imm', 0x5A)
            a.op('STA', 'abs', 0x2007); a.op('INY'); a.op('BNE', 'rel', f'up{half}_{page}')
    a.op('LDA', 'imm', 0x0E); a.op('STA', 'zp', MMC1_CTRL)
    a.op('LDA', 'zp', CTRL_SHADOW); a.op('STA', 'abs', 0x2000); a.op('LDA', 'imm', 0x1E); a.op('STA', 'abs', 0x2001)
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 0x07); a.op('CMP', 'imm', 7)
    a.op('BCC', 'rel', 'bk_ok'); a.op('LDA', 'imm', 3)
    a.label('bk_ok')
    a.op('STA', 'zp', BANK); _mmc1_write(a, 0xE000)
    a.op('JSR', 'abs', 0x8000)
    _filler(a, rng, blocks, 'f', 't_mix', with_prg_ram=True)
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x1F); a.op('BNE', 'rel', 'no_mir')
    a.op('LDA', 'zp', MMC1_CTRL); a.op('EOR', 'imm', 0x01); a.op('STA', 'zp', MMC1_CTRL); _mmc1_write(a, 0x8000)   # V <-> H
    a.label('no_mir')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    # one CHR RAM tile per frame: tile (FRAMES & 63) of pattern table 0 from the tile table, shifted by the frame
    a.op('LDA', 'abs', 0x2002)
    a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 0x3F); a.op('LSR', 'acc'); a.op('LSR', 'acc'); a.op('LSR', 'acc')
    a.op('LSR', 'acc'); a.op('STA', 'abs', 0x2006)
    a.op('LDA', 'zp', FRAMES); a.op('ASL', 'acc'); a.op('ASL', 'acc'); a.op('ASL', 'acc'); a.op('ASL', 'acc')
    a.op('STA', 'abs', 0x2006)
    a.op('LDX', 'imm', 16); a.op('LDY', 'zp', FRAMES)
    a.label('tile')
    a.op('LDA', 'aby', 0xD000); a.op('STA', 'abs', 0x2007); a.op('INY'); a.op('DEX'); a.op('BNE', 'rel', 'tile')
    a.op('LDA', 'zp', PX); a.op('STA', 'abs', 0x2005); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2005)
    a.op('LDA', 'zp', CTRL_SHADOW); a.op('STA', 'abs', 0x2000)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    code = a.assemble()
    assert len(code) <= 0x1FFA, len(code)
    fixed = bytearray(16384)
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        off = a.labels[name] - 0xC000
        fixed[off:off + len(t)] = bytes(int(v) for v in t)
    fixed[0x1000:0x2000] = tiles.tobytes()
    fixed[0x2000:0x2000 + len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    fixed[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    return ines(b''.join(banks) + bytes(fixed), b'', 1, vertical=True)


SEAM_LOOPS, SEAM_JMP, SEAM_HEADS, SEAM_RAM, SEAM_TAILS, SEAM_BANK2, SEAM_MODE = 0x70, 0x71, 0x72, 0x73, 0x74, 0x75, 0x76
SEAM_VEC = 0x04FF                         # JMP ($04FF): the 6502 takes the high byte from $0400
SEAM_RAM_CODE = 0x0500                    # the routine copied to CPU RAM


def _seam_run(a: Asm, rng: np.random.Generator, last: int, strip: int):
    """Instructions filling a.pc .. a.pc + 15 exactly, the last one `last` bytes long: the bytes that run off the end
    of an 8 KB window into the next one. A two-byte slot may be a branch into the next window's landing strip."""
    end = a.pc + 16
    while a.pc < end:
        room = end - a.pc
        n = last if room == last else int(rng.integers(1, min(3, room - last) + 1)) if room > last else room
        if n == 1:
            a.op(('NOP', 'INX', 'DEY', 'CLC', 'SEC')[int(rng.integers(5))])
        elif n == 2:
            k = int(rng.integers(5))
            if k == 4:
                a.op('BCC', 'rel', strip + int(rng.integers(8)))
            else:
                a.op(*(('LDA', 'zp'), ('ADC', 'imm'), ('STA', 'zp'), ('EOR', 'imm'))[k],
                     int(rng.choice(SCRATCH_ZP)) if k in (0, 2) else int(rng.integers(256)))
        else:
            k = int(rng.integers(4))
            a.op(('LDA', 'STA', 'INC', 'ADC')[k], 'abs', WORK_PAGE + int(rng.integers(256)) if k < 3 else 0xE300
                 + int(rng.integers(256)))


def seam_cart(seed: int = 0, blocks: int = 8, sub_blocks: int = 6) -> bytes:
    """MMC3 cartridge whose code crosses its 8 KB PRG windows in every way a program can: 128 KB PRG (16 x 8 KB;
    banks 0-14 share one layout, bank 15 is fixed at $E000 with the main loop, the tables and the vectors), 128 KB
    random CHR. Each of banks 0-14 starts with a head (a 16-NOP landing strip at offset 0, then code that loops back
    into the previous window and returns) and ends with a tail (offset $1F80: an entry that may branch forward into
    the next window's strip, seeded work, a 16-NOP strip at $1FE0, then 16 bytes of 1-, 2- and 3-byte instructions
    ending exactly on the window's last byte, the last one's length differing between banks, which run into the next
    window). The main loop maps two banks (R6, R7, possibly the same one) in PRG mode 0 or 1, so a tail at $8000 or
    $A000 runs into a head at $A000 or $C000 of another bank (bank 14 in the fixed slot included); it enters the tail
    by JSR or by JMP ($04FF) (the vector's high byte from $0400, the 6502's page wrap), loops through the seam 1-4
    times, and calls a routine copied to CPU RAM at $0500 that calls back into PRG. Every pass counts itself in zero
    page (heads $72, RAM routine $73, tails $74)."""
    rng = np.random.default_rng([0x5345414D, seed])
    pal, nt, oam, mix = _tables(rng)
    # fixed bank 15 at $E000: tables, main loop, NMI, helper; the RAM routine's image at $FF00
    a = Asm(0xE000)
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    assert a.labels['t_mix'] == 0xE220
    a.data(rng.integers(0, 256, 256, dtype=np.uint8).tobytes())        # $E300: a table the seam runs read
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    a.op('LDA', 'imm', 0x80); a.op('STA', 'abs', 0xA001)               # PRG RAM on
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0xA000)                  # vertical mirroring
    _reset_common(a, 0x88, tables)
    a.op('LDX', 'imm', 0)
    a.label('cp'); a.op('LDA', 'abx', 0xFF00); a.op('STA', 'abx', SEAM_RAM_CODE); a.op('INX'); a.op('CPX', 'imm', 32)
    a.op('BNE', 'rel', 'cp')
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    for var, shift, lab in ((BANK, 0, 'b6'), (SEAM_BANK2, 3, 'b7')):   # two banks of 0-14
        a.op('LDA', 'zp', CNT_LO)
        for _ in range(shift):
            a.op('LSR', 'acc')
        a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 0x0F); a.op('CMP', 'imm', 15); a.op('BCC', 'rel', lab)
        a.op('LDA', 'zp', FRAMES); a.op('AND', 'imm', 7)
        a.label(lab); a.op('STA', 'zp', var)
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', FRAMES); a.op('AND', 'imm', 0x10); a.op('ASL', 'acc'); a.op('ASL', 'acc')
    a.op('STA', 'zp', SEAM_MODE)                                        # PRG mode bit 6
    a.op('ORA', 'imm', 6); a.op('STA', 'abs', 0x8000); a.op('LDA', 'zp', BANK); a.op('STA', 'abs', 0x8001)
    a.op('LDA', 'zp', SEAM_MODE); a.op('ORA', 'imm', 7); a.op('STA', 'abs', 0x8000)
    a.op('LDA', 'zp', SEAM_BANK2); a.op('STA', 'abs', 0x8001)
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 3); a.op('CLC'); a.op('ADC', 'imm', 1); a.op('STA', 'zp', SEAM_LOOPS)
    a.op('LDA', 'imm', 0x80); a.op('STA', 'abs', SEAM_VEC)               # the tail entry of window $8000 or $A000
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x40); a.op('BEQ', 'rel', 'w8')
    a.op('LDA', 'imm', 0xBF); a.op('BNE', 'rel', 'wset')
    a.label('w8'); a.op('LDA', 'imm', 0x9F)
    a.label('wset'); a.op('STA', 'abs', SEAM_VEC + 1 - 0x100)
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 0x20); a.op('BEQ', 'rel', 'by_jsr')
    a.op('LDA', 'imm', 1); a.op('STA', 'zp', SEAM_JMP); a.op('JMP', 'ind', SEAM_VEC)
    a.label('by_jsr')
    a.op('LDA', 'imm', 0); a.op('STA', 'zp', SEAM_JMP)
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x40); a.op('BEQ', 'rel', 'j8')
    a.op('JSR', 'abs', 0xBF80); a.op('JMP', 'abs', 'main_ret')
    a.label('j8'); a.op('JSR', 'abs', 0x9F80)
    a.label('main_ret')
    a.op('JSR', 'abs', SEAM_RAM_CODE)
    _filler(a, rng, blocks, 'f', 't_mix', with_prg_ram=True)
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    a.label('helper')
    a.op('LDA', 'zp', 0x58); a.op('CLC'); a.op('ADC', 'imm', 0x11); a.op('STA', 'zp', 0x58); a.op('RTS')
    code_e = a.assemble()
    assert len(code_e) <= 0x1F00, len(code_e)
    r = Asm(SEAM_RAM_CODE)                                              # runs from CPU RAM
    r.op('INC', 'zp', SEAM_RAM); r.op('LDA', 'zp', SEAM_RAM); r.op('EOR', 'zp', PAD); r.op('STA', 'zp', 0x5E)
    r.op('JSR', 'abs', a.labels['helper']); r.op('AND', 'imm', 7); r.op('BNE', 'rel', 'r_out'); r.op('INC', 'zp', 0x5D)
    r.label('r_out'); r.op('RTS')
    ram_code = r.assemble()
    assert len(ram_code) <= 32
    fixed = bytearray(8192)
    fixed[:len(code_e)] = code_e
    fixed[0x1F00:0x1F00 + len(ram_code)] = ram_code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    fixed[0x1FFA:0x2000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    banks = []
    for b in range(15):
        page = bytearray(8192)
        h = Asm(0xA000)                                                 # head (position independent)
        for _ in range(16):
            h.op('NOP')
        h.op('DEC', 'zp', SEAM_LOOPS); h.op('BEQ', 'rel', 'h_done'); h.op('LDA', 'zp', SEAM_LOOPS)
        h.op('BNE', 'rel', 0x9FE0 + int(rng.integers(16)))              # back into the previous window's strip
        h.label('h_done')
        h.op('INC', 'zp', SEAM_HEADS); h.op('JSR', 'abs', a.labels['helper'])
        _filler(h, rng, sub_blocks, f'h{b}', 0xE300, with_prg_ram=True)
        h.op('LDA', 'zp', SEAM_JMP); h.op('BNE', 'rel', 'hx'); h.op('RTS')
        h.label('hx'); h.op('JMP', 'abs', a.labels['main_ret'])
        head = h.assemble()
        page[:len(head)] = head
        t = Asm(0x9F80)                                                 # tail (position independent)
        t.op('INC', 'zp', SEAM_TAILS); t.op('LDA', 'zp', PAD); t.op('AND', 'imm', 1 << int(rng.integers(8)))
        t.op('BNE', 'rel', 0xA000 + int(rng.integers(8)))               # forward into the next window's strip
        while True:                                                     # seeded work up to the strip at $1FE0
            w = Asm(t.pc)
            _filler(w, rng, 1, f't{b}_{t.pc:x}', 0xE300, with_prg_ram=True)
            if w.pc > 0x9FE0:
                break
            t.items += w.items
            t.labels.update(w.labels)
            t.pc = w.pc
        while t.pc < 0x9FE0:
            t.op('NOP')
        for _ in range(16):
            t.op('NOP')
        _seam_run(t, rng, b % 3 + 1, 0xA000)
        assert t.pc == 0xA000
        tail = t.assemble()
        page[0x1F80:] = tail
        assert len(head) <= 0x1F00
        banks.append(bytes(page))
    chr_ = rng.integers(0, 256, 128 * 1024, dtype=np.uint8).tobytes()
    return ines(b''.join(banks) + bytes(fixed), chr_, 4, vertical=True)


def mmc2_cart(seed: int = 0, blocks: int = 12, sub_blocks: int = 12) -> bytes:
    """MMC2 (mapper 9) cartridge: 128 KB PRG in 8 KB banks (0-12 switched in at $8000, the last three fixed at
    $A000-$FFFF), 128 KB CHR ROM in 4 KB banks. The nametables and sprites use tiles $FD and $FE often, so the
    renderer's fetches flip the latches of both pattern halves mid-line; the main loop calls a subroutine in the
    $8000 bank, rewrites the four CHR bank registers and the mirroring now and then, swaps the background and
    sprite pattern halves, and reads $0FD8/$0FE8/$1FD8/$1FE8 through $2006/$2007 (CPU-driven latch flips)."""
    rng = np.random.default_rng([0x4D4D4332, seed])
    pal, nt, oam, mix = _tables(rng)
    trig = rng.random(256) < 0.12
    nt[trig] = rng.choice(np.array([0xFD, 0xFE]), int(trig.sum()))
    tiles = oam[1::4]
    st = rng.random(64) < 0.3
    tiles[st] = rng.choice(np.array([0xFD, 0xFE]), int(st.sum()))
    oam[1::4] = tiles
    banks = []
    for b in range(13):   # switchable: a subroutine at $8000, a table at $9F00
        sub = Asm(0x8000)
        _filler(sub, rng, sub_blocks, f'b{b}', 0x9F00)
        sub.op('RTS')
        body = sub.assemble()
        assert len(body) <= 0x1F00, len(body)
        page = bytearray(8192)
        page[:len(body)] = body
        page[0x1F00:0x2000] = rng.integers(0, 256, 256, dtype=np.uint8).tobytes()
        banks.append(bytes(page))
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)                                        # NMI on, BG at $1000, sprites at $0000
    a.label('main')
    _read_pad(a, 'm')
    _pad_moves(a, 't_mix')
    a.op('LDA', 'zp', CNT_LO); a.op('EOR', 'zp', PAD); a.op('AND', 'imm', 0x07); a.op('STA', 'zp', BANK)
    a.op('STA', 'abs', 0xA000); a.op('JSR', 'abs', 0x8000)
    _filler(a, rng, blocks, 'f', 't_mix')
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x0F); a.op('BNE', 'rel', 'no_chr')
    a.op('LDA', 'zp', CNT_HI); a.op('EOR', 'zp', PX)
    for k, reg in enumerate((0xB000, 0xC000, 0xD000, 0xE000)):
        a.op('STA', 'abs', reg); a.op('CLC'); a.op('ADC', 'imm', 7 + 2 * k)
    a.label('no_chr')
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x1F); a.op('CMP', 'imm', 5); a.op('BNE', 'rel', 'no_mir')
    a.op('LDA', 'zp', CNT_HI); a.op('STA', 'abs', 0xF000)
    a.label('no_mir')
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x3F); a.op('CMP', 'imm', 9); a.op('BNE', 'rel', 'no_swap')
    a.op('LDA', 'zp', CTRL_SHADOW); a.op('EOR', 'imm', 0x18); a.op('STA', 'zp', CTRL_SHADOW)   # swap the halves
    a.label('no_swap')
    a.op('LDA', 'zp', CNT_LO); a.op('AND', 'imm', 0x0F); a.op('CMP', 'imm', 3); a.op('BNE', 'rel', 'no_cpu')
    a.op('LDA', 'abs', 0x2002)                                            # CPU-driven latch flips
    a.op('LDA', 'zp', CNT_HI); a.op('AND', 'imm', 0x10); a.op('ORA', 'imm', 0x0F); a.op('STA', 'abs', 0x2006)
    a.op('LDA', 'zp', PX); a.op('AND', 'imm', 0x10); a.op('ORA', 'imm', 0xD8); a.op('STA', 'abs', 0x2006)
    a.op('LDA', 'abs', 0x2007); a.op('LDA', 'abs', 0x2007)
    a.label('no_cpu')
    a.op('JMP', 'abs', 'main')
    a.label('nmi')
    _nmi_common(a)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    assert len(code) <= 0x3FFA, len(code)
    fixed = bytearray(24576)                                              # banks 13-15 at $A000-$FFFF
    fixed[0x2000:0x2000 + len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    fixed[0x5FFA:0x6000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 131072, dtype=np.uint8).tobytes()
    return ines(b''.join(banks) + bytes(fixed), chr_, 9, vertical=True)


DCNT, DYCNT = 0x44, 0x45                  # frames Down has been held, frames spent dying


def smb_like_cart(seed: int = 0) -> bytes:
    """NROM-128 cartridge that plays like the SMB reward reader expects (it writes the reader's RAM bytes), so the
    env's reward, death, level and game-over paths all run. SMB's structure: the main loop is a JMP-to-self idle
    loop and everything happens in the NMI (OAM DMA, nametable and scroll writes, pad read, game logic).

    In play (mode $0770 = 1, task $0772 = 3, routine $0E = 8): Right moves the position ($6D page, $86 x) 2 px
    forward, Left 1 px back, A adds 10 points (score digits $07E1-$07E2), holding Down for 24 frames starts dying
    (routine 6); page 3 is the next level ($075C, then world $075F), world 8 wins (mode 2, world 7). Dying lasts 30
    frames, then a life ($075A) is lost and play resumes at the level start; losing a life at 0 is game over
    (mode 3). Like SMB, the NMI ends with the status-bar split: it waits for the sprite-0 hit (sprite 0 at line
    24) and then writes the horizontal scroll, mid-line."""
    rng = np.random.default_rng([0x534D424C, seed])
    pal, nt, oam, mix = _tables(rng)
    oam[0:4] = (23, int(oam[1]), 0x00, 88)                    # sprite 0 at the bottom of a status bar, as in SMB
    a = Asm(0xC000)
    tables = dict(pal='t_pal', nt='t_nt', oam='t_oam')
    a.label('reset')
    _reset_common(a, 0x90, tables)
    for addr, v in ((0x0770, 1), (0x0772, 3), (0x000E, 8), (0x075A, 2), (0x0086, 40)):
        a.op('LDA', 'imm', v); a.op('STA', 'abs', addr)
    a.label('idle')
    a.op('JMP', 'abs', 'idle')
    a.label('nmi')
    _nmi_common(a)
    _read_pad(a, 'n')
    a.op('LDA', 'abs', 0x0770); a.op('CMP', 'imm', 1); a.op('BEQ', 'rel', 'inplay'); a.op('JMP', 'abs', 'done')
    a.label('inplay')
    a.op('LDA', 'zp', 0x0E); a.op('CMP', 'imm', 8); a.op('BEQ', 'rel', 'alive'); a.op('JMP', 'abs', 'dying')
    a.label('alive')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x80); a.op('BEQ', 'rel', 'noright')
    a.op('LDA', 'zp', 0x86); a.op('CLC'); a.op('ADC', 'imm', 2); a.op('STA', 'zp', 0x86)
    a.op('LDA', 'zp', 0x6D); a.op('ADC', 'imm', 0); a.op('STA', 'zp', 0x6D)
    a.label('noright')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x40); a.op('BEQ', 'rel', 'noleft')
    a.op('LDA', 'zp', 0x86); a.op('SEC'); a.op('SBC', 'imm', 1); a.op('STA', 'zp', 0x86)
    a.op('LDA', 'zp', 0x6D); a.op('SBC', 'imm', 0); a.op('STA', 'zp', 0x6D)
    a.label('noleft')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x01); a.op('BEQ', 'rel', 'noa')
    a.op('INC', 'abs', 0x07E2); a.op('LDA', 'abs', 0x07E2); a.op('CMP', 'imm', 10); a.op('BCC', 'rel', 'noa')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x07E2); a.op('INC', 'abs', 0x07E1)
    a.label('noa')
    a.op('LDA', 'zp', PAD); a.op('AND', 'imm', 0x20); a.op('BEQ', 'rel', 'nodown')
    a.op('INC', 'zp', DCNT); a.op('LDA', 'zp', DCNT); a.op('CMP', 'imm', 24); a.op('BCC', 'rel', 'moved')
    a.op('LDA', 'imm', 6); a.op('STA', 'zp', 0x0E); a.op('LDA', 'imm', 0); a.op('STA', 'zp', DCNT)
    a.op('JMP', 'abs', 'done')
    a.label('nodown')
    a.op('LDA', 'imm', 0); a.op('STA', 'zp', DCNT)
    a.label('moved')
    a.op('LDA', 'zp', 0x6D); a.op('BMI', 'rel', 'done_n'); a.op('CMP', 'imm', 3); a.op('BCC', 'rel', 'done_n')
    a.op('INC', 'abs', 0x075C); a.op('LDA', 'imm', 0); a.op('STA', 'zp', 0x6D); a.op('LDA', 'imm', 40)
    a.op('STA', 'zp', 0x86)
    a.op('LDA', 'abs', 0x075C); a.op('CMP', 'imm', 4); a.op('BCC', 'rel', 'done_n')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x075C); a.op('INC', 'abs', 0x075F)
    a.op('LDA', 'abs', 0x075F); a.op('CMP', 'imm', 8); a.op('BCC', 'rel', 'done_n')
    a.op('LDA', 'imm', 7); a.op('STA', 'abs', 0x075F); a.op('LDA', 'imm', 2); a.op('STA', 'abs', 0x0770)
    a.label('done_n')
    a.op('JMP', 'abs', 'done')
    a.label('dying')
    a.op('INC', 'zp', DYCNT); a.op('LDA', 'zp', DYCNT); a.op('CMP', 'imm', 30); a.op('BCC', 'rel', 'done')
    a.op('LDA', 'imm', 0); a.op('STA', 'zp', DYCNT); a.op('LDA', 'imm', 8); a.op('STA', 'zp', 0x0E)
    a.op('LDA', 'imm', 0); a.op('STA', 'zp', 0x6D); a.op('LDA', 'imm', 40); a.op('STA', 'zp', 0x86)
    a.op('DEC', 'abs', 0x075A); a.op('BPL', 'rel', 'done')
    a.op('LDA', 'imm', 3); a.op('STA', 'abs', 0x0770)
    a.label('done')
    # SMB's status-bar split: wait for the sprite-0 flag to drop (pre-render line), then for the hit, a short delay
    # into the line, then the playfield's horizontal scroll (each wait bounded)
    a.op('LDX', 'imm', 0)
    a.label('s0c'); a.op('BIT', 'abs', 0x2002); a.op('BVC', 'rel', 's0c_ok'); a.op('DEX'); a.op('BNE', 'rel', 's0c')
    a.label('s0c_ok')
    a.op('LDY', 'imm', 4)
    a.label('s0w'); a.op('BIT', 'abs', 0x2002); a.op('BVS', 'rel', 's0h'); a.op('DEX'); a.op('BNE', 'rel', 's0w')
    a.op('DEY'); a.op('BNE', 'rel', 's0w')
    a.label('s0h')
    a.op('LDY', 'imm', 5)
    a.label('s0d'); a.op('DEY'); a.op('BNE', 'rel', 's0d')
    a.op('LDA', 'zp', 0x86); a.op('STA', 'abs', 0x2005); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2005)
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_mix', mix)):
        a.label(name)
        a.data(bytes(int(v) for v in t))
    code = a.assemble()
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


SPEC_PAD, SPEC_PTR, SPEC_RNG = 0xE0, 0xE2, 0xE4   # zero page of spec_cart (no reward reader reads $E0-$E7)


def spec_cart(spec: dict, seed: int = 0) -> bytes:
    """NROM-128 cartridge that drives a reward reader's RAM bytes from the pad, so a game's reader (any of the
    reward10 games) sees play, deaths, level changes and game overs inside the env. spec: RAM address -> list of
    values, or ('walk', lo, hi, step). The main loop idles; each NMI does OAM DMA, reads the pad into $E0 and
    visits the spec entries in order: a list entry takes a value drawn from its list with p ~1/32 per frame (a
    16-bit xorshift at $E4/$E5, its low byte mixed with the pad each frame, draws); a walk moves by its step
    towards hi while Right is held, towards lo while Left is held, else one random step with p 1/8, clamped to
    [lo, hi]."""
    rng = np.random.default_rng([0x53504543, seed])
    pal, nt, oam, _ = _tables(rng)
    entries = sorted(spec.items())
    assert 0 < len(entries) <= 255 and all(not (0xE0 <= a <= 0xE7) and a < 0x800 for a, _ in entries)
    lo_t, hi_t, kind_t, ta, tb, tc, pool = [], [], [], [], [], [], []
    for addr, c in entries:
        lo_t.append(addr & 0xFF)
        hi_t.append(addr >> 8)
        if isinstance(c, list):
            assert 0 < len(c) <= 16
            kind_t.append(0); ta.append(len(c)); tb.append(len(pool)); tc.append(0)
            pool += c
        else:
            _, lo, hi, step = c
            kind_t.append(1); ta.append(lo); tb.append(hi); tc.append(step)
    assert len(pool) + 16 <= 256
    a = Asm(0xC000)
    a.label('reset')
    _reset_common(a, 0x90, dict(pal='t_pal', nt='t_nt', oam='t_oam'))
    a.op('LDA', 'imm', 0x5A); a.op('STA', 'zp', SPEC_RNG); a.op('LDA', 'imm', 0xC3); a.op('STA', 'zp', SPEC_RNG + 1)
    for addr, c in entries:
        a.op('LDA', 'imm', c[0] if isinstance(c, list) else (c[1] + c[2]) // 2); a.op('STA', 'abs', addr)
    a.label('idle')
    a.op('JMP', 'abs', 'idle')
    a.label('rng')   # 16-bit xorshift (7, 9, 8) at $E4/$E5; A = the high byte
    a.op('LDA', 'zp', SPEC_RNG + 1); a.op('LSR', 'acc'); a.op('LDA', 'zp', SPEC_RNG); a.op('ROR', 'acc')
    a.op('EOR', 'zp', SPEC_RNG + 1); a.op('STA', 'zp', SPEC_RNG + 1); a.op('ROR', 'acc'); a.op('EOR', 'zp', SPEC_RNG)
    a.op('STA', 'zp', SPEC_RNG); a.op('EOR', 'zp', SPEC_RNG + 1); a.op('STA', 'zp', SPEC_RNG + 1); a.op('RTS')
    a.label('nmi')
    a.op('PHA'); a.op('TXA'); a.op('PHA'); a.op('TYA'); a.op('PHA')
    a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x2003); a.op('LDA', 'imm', OAM_PAGE >> 8); a.op('STA', 'abs', 0x4014)
    a.op('LDA', 'imm', 1); a.op('STA', 'abs', 0x4016); a.op('LDA', 'imm', 0); a.op('STA', 'abs', 0x4016)
    a.op('LDX', 'imm', 8)
    a.label('sprd')
    a.op('LDA', 'abs', 0x4016); a.op('LSR', 'acc'); a.op('ROR', 'zp', SPEC_PAD); a.op('DEX'); a.op('BNE', 'rel', 'sprd')
    a.op('LDA', 'zp', SPEC_RNG); a.op('EOR', 'zp', SPEC_PAD); a.op('STA', 'zp', SPEC_RNG); a.op('ORA', 'zp', SPEC_RNG + 1)
    a.op('BNE', 'rel', 'seed_ok'); a.op('INC', 'zp', SPEC_RNG)   # the all-zero state would stay zero
    a.label('seed_ok')
    a.op('LDX', 'imm', 0)
    a.label('ent')
    a.op('LDA', 'abx', 't_lo'); a.op('STA', 'zp', SPEC_PTR); a.op('LDA', 'abx', 't_hi'); a.op('STA', 'zp', SPEC_PTR + 1)
    a.op('LDA', 'abx', 't_kind'); a.op('BNE', 'rel', 'walk')
    # list: p 1/32, then an index below the list length (drawn in 0..15, out of range = no change)
    a.op('JSR', 'abs', 'rng'); a.op('AND', 'imm', 31); a.op('BNE', 'rel', 'next_n')
    a.op('JSR', 'abs', 'rng'); a.op('AND', 'imm', 15); a.op('CMP', 'abx', 't_a'); a.op('BCS', 'rel', 'next_n')
    a.op('CLC'); a.op('ADC', 'abx', 't_b'); a.op('TAY'); a.op('LDA', 'aby', 't_pool'); a.op('JMP', 'abs', 'store')
    a.label('next_n')
    a.op('JMP', 'abs', 'next')
    a.label('walk')
    a.op('LDY', 'imm', 0)
    a.op('LDA', 'zp', SPEC_PAD); a.op('AND', 'imm', 0x80); a.op('BNE', 'rel', 'up')
    a.op('LDA', 'zp', SPEC_PAD); a.op('AND', 'imm', 0x40); a.op('BNE', 'rel', 'down')
    a.op('JSR', 'abs', 'rng'); a.op('AND', 'imm', 7); a.op('BNE', 'rel', 'next_n')
    a.op('JSR', 'abs', 'rng'); a.op('AND', 'imm', 1); a.op('BEQ', 'rel', 'down')
    a.label('up')
    a.op('LDY', 'imm', 0); a.op('LDA', 'izy', SPEC_PTR); a.op('CLC'); a.op('ADC', 'abx', 't_c'); a.op('BCS', 'rel', 'to_hi')
    a.op('CMP', 'abx', 't_b'); a.op('BCC', 'rel', 'store'); a.op('BEQ', 'rel', 'store')
    a.label('to_hi')
    a.op('LDA', 'abx', 't_b'); a.op('JMP', 'abs', 'store')
    a.label('down')
    a.op('LDY', 'imm', 0); a.op('LDA', 'izy', SPEC_PTR); a.op('SEC'); a.op('SBC', 'abx', 't_c'); a.op('BCC', 'rel', 'to_lo')
    a.op('CMP', 'abx', 't_a'); a.op('BCS', 'rel', 'store')
    a.label('to_lo')
    a.op('LDA', 'abx', 't_a')
    a.label('store')
    a.op('LDY', 'imm', 0); a.op('STA', 'izy', SPEC_PTR)
    a.label('next')
    a.op('INX'); a.op('CPX', 'imm', len(entries)); a.op('BEQ', 'rel', 'out'); a.op('JMP', 'abs', 'ent')
    a.label('out')
    _nmi_end(a)
    a.label('irq')
    a.op('RTI')
    for name, t in (('t_pal', pal), ('t_nt', nt), ('t_oam', oam), ('t_lo', lo_t), ('t_hi', hi_t),
                    ('t_kind', kind_t), ('t_a', ta), ('t_b', tb), ('t_c', tc), ('t_pool', pool + [0] * 16)):
        a.label(name)
        a.data(bytes(int(v) & 0xFF for v in t))
    code = a.assemble()
    prg = bytearray(16384)
    prg[:len(code)] = code
    vec = (a.labels['nmi'], a.labels['reset'], a.labels['irq'])
    prg[0x3FFA:0x4000] = bytes(sum(((v & 0xFF, v >> 8) for v in vec), ()))
    chr_ = rng.integers(0, 256, 8192, dtype=np.uint8).tobytes()
    return ines(bytes(prg), chr_, 0, vertical=True)


# ------------------------------------------------------------------------------- SMB RAM trajectories

SMB_ADDRS = (0x0E, 0x6D, 0x86, 0xB5, 0x75A, 0x75C, 0x75F, 0x770, 0x772, 0x7DD, 0x7DE, 0x7DF, 0x7E0, 0x7E1, 0x7E2)


def smb_ram15(seed: int, n_envs: int, steps: int) -> np.ndarray:
    """uint8 [steps, n_envs, 16]: per env-step the SMB reader's 15 RAM bytes (SMB_ADDRS order), byte 15 = 0."""
    rng = np.random.default_rng([0x534D4252, seed])
    n = n_envs
    x = np.full(n, 40, np.int64)
    world = np.zeros(n, np.int64)
    level = np.zeros(n, np.int64)
    lives = np.full(n, 2, np.int64)
    score = np.zeros(n, np.int64)       # in units of 10 points
    mode = np.ones(n, np.int64)
    out = np.zeros((steps, n, 16), np.uint8)
    for t in range(steps):
        u = rng.random((n, 6))
        step = rng.integers(1, 5, n) * np.where(u[:, 0] < 0.8, 1, -1)
        x = np.clip(x + step, 0, 0x7FFF)
        back = u[:, 1] < 0.05                      # a one-step excursion back (a rollback when x >= ~760)
        x_obs = np.where(back, np.maximum(x - rng.integers(760, 1400, n), 0), x)
        adv = u[:, 2] < 1e-3
        level = np.where(adv, level + 1, level)
        world = np.where(adv & (level == 4), np.minimum(world + 1, 7), world)
        level = np.where(level == 4, 0, level)
        x = np.where(adv, 40, x)
        die = u[:, 3] < 5e-4
        lives = np.where(die, lives - 1, lives)
        mode = np.where(lives < 0, 3, mode)
        mode = np.where(adv & (world == 7) & (level == 3), 2, mode)
        score = np.where(u[:, 4] < 0.1, score + rng.integers(1, 20, n), score) % 1000000
        pit = u[:, 5] < 1e-4
        routine = np.where(die, 6, 8)
        b5 = np.where(pit, 2, 1)
        digits = [(score // 10 ** (5 - k)) % 10 for k in range(6)]
        cols = [routine, (x_obs >> 8) & 0xFF, x_obs & 0xFF, b5, lives & 0xFF, level, world, mode,
                np.full(n, 3)] + digits
        out[t, :, :15] = np.stack(cols, axis=1).astype(np.uint8)
    return out


def expand_ram(ram15: np.ndarray) -> np.ndarray:
    """[..., 16] packed bytes -> [..., 2048] RAM images with the 15 bytes at their addresses, zeros elsewhere."""
    full = np.zeros(ram15.shape[:-1] + (2048,), np.uint8)
    for i, a in enumerate(SMB_ADDRS):
        full[..., a] = ram15[..., i]
    return full
