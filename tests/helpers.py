"""Shared test helpers: library paths, the oracle's extra entry points, record field access."""
from __future__ import annotations

import ctypes
import struct
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_LIB = ROOT / 'oracle' / '_build' / 'liboracle_rlenv.so'
HIP_LIB = ROOT / 'ghostrun-lab_amd' / 'csrc' / '_build' / 'librlenv_hip.so'
GOLDEN = ROOT / 'tests' / 'golden'
REC_BYTES = 23552

# NesRec field offsets (include/nesrec.h)
OFF = dict(pc=0x00, a=0x02, x=0x03, y=0x04, sp=0x05, p=0x06, irq_line=0x07, cycles=0x08, nmi_pending=0x10, pad=0x11,
           shift=0x12, strobe=0x13, instr=0x14, frame_dot=0x18, frame=0x1C, v=0x20, t=0x22, ctrl=0x24, mask=0x25,
           status=0x26, oam_addr=0x27, fx=0x28, w=0x29, read_buf=0x2A, open_bus=0x2B, s0_sched=0x2C, log_frame=0x30,
           log_n=0x34, log_flags=0x36, dmc_byte_end=0x40, dmc_event=0x48, dmc_left=0x50, ram=0x100, nt=0x900,
           oam=0x1100, pal=0x1200, log=0x1300, prg_ram=0x1C00, chr_ram=0x3C00, mreg=0x58, prg_off=0x68, chr_off=0x78,
           nt_map=0x98)

_oracle = None


def oracle():
    """The CPU oracle library with its extra test entry points bound."""
    global _oracle
    if _oracle is None:
        lib = ctypes.CDLL(str(ORACLE_LIB))
        P, I, U64, U32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32
        lib.orc_rl10_replay.argtypes = [I, P, I, P, P, P, P, P, P, P]
        lib.orc_pad_table.argtypes = [P]
        lib.orc_legal_table.argtypes = [I, I, P, P]
        lib.orc_schedule.argtypes = [U64, I, I, P, P, U32]
        lib.orc_episode_seed.argtypes = [U64, U32, U64]
        lib.orc_episode_seed.restype = U64
        lib.orc_rl10_step.argtypes = [P, P, I, P, I, P]
        lib.orc_smb_observe.argtypes = [P, P]
        lib.orc_power_on.argtypes = [P, P]
        lib.orc_run_until.argtypes = [P, P, U64]
        lib.orc_run_until.restype = U32
        lib.orc_step.argtypes = [P, P, P]
        lib.orc_step.restype = U32
        lib.orc_render_full.argtypes = [P, P, P, P]
        lib.orc_render_obs.argtypes = [P, P, P, P]
        lib.orc_bus_read.argtypes = [P, P, ctypes.c_uint16]
        lib.orc_bus_read.restype = ctypes.c_uint8
        lib.orc_bus_write.argtypes = [P, P, ctypes.c_uint16, ctypes.c_uint8]
        lib.orc_dmc_service.argtypes = [P, U64, I]
        lib.orc_dmc_service.restype = U32
        lib.orc_dmc_reset.argtypes = [P, U64]
        lib.orc_sprite0_hit.argtypes = [P, P, P]
        lib.orc_sprite0_hit.restype = U32
        lib.orc_mmc2_resolve.argtypes = [P, P]
        lib.orc_run_until_budget.argtypes = [P, P, U64, U32]
        lib.orc_run_until_budget.restype = U32
        lib.orc_ram_hash.argtypes = [P]
        lib.orc_ram_hash.restype = U64
        lib.orc_parse_ines.argtypes = [P, U32, P, U32, P, ctypes.c_char_p, I]
        lib.orc_num_threads.restype = I
        lib.rl_pack6.argtypes = [P, P, ctypes.c_size_t, P]
        lib.rl_unpack6.argtypes = [P, P, ctypes.c_size_t, P]
        lib.rl10_smb_run.argtypes = [P, I, I, I, P, P, P, P]
        lib.rl10_run.argtypes = [I, P, I, I] + [P] * 11
        _oracle = lib
    return _oracle


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if isinstance(a, np.ndarray) else ctypes.c_void_p(ctypes.addressof(a))


class NesCart(ctypes.Structure):
    _fields_ = [('prg', ctypes.c_void_p), ('prg_size', ctypes.c_uint32), ('chr', ctypes.c_void_p),
                ('chr_size', ctypes.c_uint32), ('board', ctypes.c_uint8), ('mirroring', ctypes.c_uint8)]


class Console:
    """One oracle console on a cartridge: record bytes + the cart view (for unit tests of the machine)."""

    def __init__(self, rom: bytes):
        self.lib = oracle()
        self.rom = np.frombuffer(bytes(rom), np.uint8).copy()
        self.prg = np.zeros(1 << 20, np.uint8)
        self.cart = NesCart()
        err = ctypes.create_string_buffer(256)
        if self.lib.orc_parse_ines(ptr(self.rom), len(self.rom), ptr(self.prg), len(self.prg), ptr(self.cart), err, 256):
            raise ValueError(err.value.decode())
        self.rec = np.zeros(REC_BYTES, np.uint8)
        self.lib.orc_power_on(ptr(self.rec), ptr(self.cart))

    def cart_ptr(self):
        return ptr(self.cart)

    def u(self, name, fmt='B'):
        return struct.unpack_from('<' + fmt, self.rec, OFF[name])[0]

    def set(self, name, value, fmt='B'):
        struct.pack_into('<' + fmt, self.rec, OFF[name], value)

    def step(self):
        fault = ctypes.c_uint32(0)
        cyc = self.lib.orc_step(ptr(self.rec), ptr(self.cart), ctypes.byref(fault))
        return cyc, fault.value

    def run_until(self, target):
        return self.lib.orc_run_until(ptr(self.rec), ptr(self.cart), target)

    def ram(self):
        return self.rec[OFF['ram']:OFF['ram'] + 2048]

    def read(self, addr):
        return self.lib.orc_bus_read(ptr(self.rec), ptr(self.cart), addr)

    def write(self, addr, value):
        self.lib.orc_bus_write(ptr(self.rec), ptr(self.cart), addr, value)

    def mem(self, name, n):
        return self.rec[OFF[name]:OFF[name] + n]

    def words(self, name, n):
        return self.rec[OFF[name]:OFF[name] + 4 * n].view(np.uint32)

    def render_full(self):
        pix = np.zeros((240, 256), np.uint8)
        emph = np.zeros(240, np.uint8)
        self.lib.orc_render_full(ptr(self.rec), ptr(self.cart), ptr(pix), ptr(emph))
        return pix, emph
