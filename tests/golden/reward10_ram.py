"""Seeded 2 KB RAM trajectories for the reward10 readers of the games other than SMB.

Each game lists the RAM bytes its reader reads (rl/csrc/reward10.cuh:160-507) with the values that steer the reader's
branches (the states, modes and thresholds it compares against). A trajectory starts from seeded random RAM; at each
step every listed byte keeps its value with probability 0.8 and otherwise draws a candidate, or for a walk moves by
a small step, so play, deaths, level changes, progress, rollbacks, bosses and game overs all occur. Used by
gen_golden.py (with the reference's compiled rl10_replay) and by the tests (with the oracle and the HIP library).
"""
from __future__ import annotations

import numpy as np

GAMES = ('smb', 'pacman', 'excitebike', 'contra', 'castlevania', 'gradius', 'zelda', 'tetris', 'tecmobowl', 'kage',
         'finalmission', 'punchout')


def _walk(lo, hi, step):
    return ('walk', lo, hi, step)


DIGIT = [0, 1, 2, 3, 4, 5, 6, 7, 8, 9]
BCD = [0x00, 0x01, 0x09, 0x10, 0x25, 0x50, 0x99]

SPECS = {
    'pacman': {0x3F: [4, 6, 12, 8, 10, 3], 0x48: [0, 0, 0, 1], 0x47: [0, 0, 0, 1], 0x4A: [0, 0, 1],
               0x6A: _walk(0, 200, 6), 0x68: [0, 1, 2, 3], 0x67: [3, 2, 1, 0],
               **{0x70 + i: DIGIT for i in range(6)}},
    'excitebike': {0x43: [0, 1], 0x46: [0, 1, 2], 0x47: [1, 1, 0], 0x4F: [1, 1, 1, 0, 2], 0x52: [0, 0, 1],
                   0x12: _walk(0, 255, 8), 0x4D: [0, 1], 0xF2: [0, 0, 0, 1], 0x9C: [0, 0, 0, 1, 3, 5],
                   0x3B6: [0, 10, 31, 32, 40], 0x3B1: [0, 0, 1], 0x41: [2, 3, 4, 2, 3, 0, 1],
                   0x3F3: [0, 0, 0, 1, 2]},
    'contra': {0x18: [5, 5, 5, 4], 0x1C: [0, 0, 1], 0x2C: [4, 4, 3], 0x38: [0, 0, 0, 1], 0x32: [3, 2, 1, 0],
               0x30: [0, 0, 1, 2, 3], 0x64: _walk(0, 10, 1), 0x65: _walk(0, 255, 12), 0x40: [0, 0, 1],
               **{0x528 + i: [0, 0, 0x14, 0x11, 5] for i in range(16)},
               **{0x578 + i: _walk(0, 40, 3) for i in range(16)},
               0x25: [0, 0, 1], 0x90: [1, 1, 1, 2, 0], 0x7E2: _walk(0, 255, 5), 0x7E3: [0, 0, 1]},
    'castlevania': {0x18: [5, 5, 5, 6, 7, 13], 0x19: [6, 6, 6, 5], 0x45: _walk(0, 64, 4), 0x28: [0, 0, 1, 2, 3, 6],
                    0x41: _walk(0, 7, 1), 0x40: _walk(0, 255, 16), 0x3F: _walk(0, 255, 24), 0x1A9: _walk(0, 70, 6),
                    0x22: [0, 0, 1], 0x46C: [0, 0, 8], 0x2A: [3, 2, 1], 0x7FC: BCD, 0x7FD: BCD, 0x7FE: BCD},
    'gradius': {0x00: [5, 5, 5, 4], 0x0A: [1, 1, 0], 0x1B: [0x80, 0x81, 0x80, 0xA0, 0xA1, 192, 0x40],
                0x20: [3, 2, 1, 0, 255], 0x15: [0, 0, 1], 0x19: [0, 0, 1, 2, 3], 0x3F: _walk(0, 30, 1),
                0x3E: _walk(0, 255, 12), 0x7E4: BCD, 0x7E5: BCD, 0x7E6: BCD},
    'zelda': {0x12: [5, 5, 0xB, 0x11, 4], **{a: [0, 1, 2, 3] for a in (0x657, 0x659, 0x65A, 0x65B, 0x65C, 0x65F,
                                                                       0x660, 0x661, 0x662, 0x663, 0x664, 0x665,
                                                                       0x666, 0x674, 0x675, 0x676)},
              0x66F: [0x22, 0x32, 0x21, 0x43], 0x670: [0, 0x40, 0x80, 0xFF], 0x10: [0, 1, 2],
              0xEB: _walk(0, 255, 3), 0x70: _walk(0, 255, 20), 0x84: _walk(0, 255, 20), 0x671: [0, 1, 3, 7],
              0x66D: _walk(0, 255, 5)},
    'tetris': {0xC0: [4, 4, 4, 3], 0x48: [1, 2, 3, 5, 8, 9, 10], 0xBD: [3, 3, 3, 0], 0x51: [0, 0, 1],
               0x50: BCD, 0x64: [0, 0, 1, 2], 0x58: [0, 5, 20], 0x53: BCD, 0x54: BCD, 0x55: BCD},
    'tecmobowl': {0x43: [0x00, 0x03, 0x07, 0x10, 0x14], 0x48: [0x00, 0x03, 0x07, 0x10, 0x21], 0x2C: [8, 9, 9, 12, 3],
                  0x2D: [0, 9, 9, 12, 4], 0x8D: [0, 1, 2, 3, 4, 5], 0x8B: [0, 0, 1], 0x8A: [0, 0, 1],
                  0x8F: list(range(11)), 0x49: [0, 0, 1], 0xFB: _walk(0, 255, 10), 0xFC: [4, 5, 5, 6]},
    'kage': {0x02: [0, 0, 0, 0x6B, 1], 0x40: [0, 0, 1, 2, 3, 4, 5, 7, 14, 15], 0x6F0: _walk(0, 16, 2),
             0x22: _walk(0, 255, 40), 0x23: _walk(0x10, 0xB0, 2), 0x24: _walk(0, 255, 40), 0x25: _walk(0x18, 0x60, 2),
             0x6A1: [0, 0, 8], 0x708: [0x81, 0x80, 0x88, 0], 0x798: [20, 16, 0x4F, 0], 0x7F8: _walk(0, 100, 6),
             0xAE: [0xFF, 0], 0x758: [0x10, 0], 0xD1: [0, 0, 1]},
    'finalmission': {0x02: [4, 4, 4, 3], 0x03: [0, 0, 1], 0x38: [4, 4, 4, 7, 8], 0x4F: [0, 1, 2, 3],
                     0x85: [0, 0, 0, 1], 0x0E: [0, 0, 1], 0x1E: [0, 0, 1, 2], 0x4E: _walk(0, 31, 2),
                     0x4D: [0, 0, 1], **{a: _walk(0, 40, 4) for a in range(0x4A0, 0x4C0)}, 0x1C: [0, 2, 4, 5],
                     0x8A: _walk(0, 255, 9), 0x8B: [0, 0, 1], 0x8C: [0, 0, 0, 1]},
    'punchout': {0x00: [1, 1, 1, 1, 249, 250, 251, 252, 253, 254, 0], 0x05: [0, 1, 2], 0x01: [0, 0, 1, 2, 13],
                 0x398: _walk(0, 120, 7), 0x300: [1, 1, 0], 0x391: _walk(0, 100, 8),
                 **{0x3E8 + i: DIGIT for i in range(6)}, 0x172: [0, 0, 0, 1], 0x173: [0, 0, 0, 1]},
}


def trajectory(game: str, seed: int, steps: int):
    """RAM [steps, 2048] uint8 and frames-per-update [steps] int32 of one episode of `game`."""
    rng = np.random.default_rng([0x524C3130, GAMES.index(game), seed])
    spec = SPECS[game]
    ram = rng.integers(0, 256, 2048, dtype=np.int64)
    for a, c in spec.items():
        ram[a] = c[0] if isinstance(c, list) else rng.integers(c[1], c[2] + 1)
    out = np.empty((steps, 2048), np.uint8)
    for t in range(steps):
        for a, c in spec.items():
            if rng.random() < 0.8:
                continue
            if isinstance(c, list):
                ram[a] = c[rng.integers(len(c))]
            else:
                _, lo, hi, step = c
                ram[a] = min(hi, max(lo, int(ram[a]) + int(rng.integers(-step, step + 1))))
        out[t] = ram
    frames = rng.choice(np.array([4, 4, 4, 8, 1], np.int32), steps)
    return out, frames
