"""Move ids and random legal moves.

A move id is a mixed-radix number over the controller's five parts, least significant first: the d-pad (9
choices), A (3), B (3), Start (2) and Select (2), so there are 9 * 3 * 3 * 2 * 2 = 324 ids (the move layout of
rl/csrc/controller.cuh, as rl/actions.py packs it). The env's legal-move mask holds one byte per choice, the parts'
columns side by side in the same order (19 bytes).
"""
import itertools

import torch

RADIX = (9, 3, 3, 2, 2)                                    # d-pad, A, B, Start, Select
PLACE = tuple(itertools.accumulate((1,) + RADIX[:-1], lambda a, b: a * b))    # 1, 9, 27, 81, 162
_EDGES = tuple(itertools.accumulate((0,) + RADIX))                              # 0, 9, 12, 15, 17, 19
PARTS = list(zip(_EDGES[:-1], _EDGES[1:]))                 # the mask columns of each part
MULT = list(PLACE)
NUM_MOVES = PLACE[-1] * RADIX[-1]                          # 324


def pack(parts):
    """Five tensors of part choices (any integer dtype, broadcastable) -> int16 move ids."""
    ids = torch.zeros((), dtype=torch.long)
    for choice, place in zip(parts, PLACE):
        ids = ids + choice.long() * place
    return ids.to(torch.int16)


def unpack(ids):
    """int16 (or any integer) move ids -> the five part choices as long tensors."""
    rest = ids.long()
    out = []
    for r in RADIX:
        out.append(torch.remainder(rest, r))
        rest = torch.div(rest, r, rounding_mode='floor')
    return out


def random_legal(masks, gen=None):
    """One uniformly random legal move per env: each part's choice drawn uniformly among the choices its mask
    columns allow (masks: [N, 19] uint8, at least one legal choice per part), by inverse CDF over the mask with one
    uniform draw per env and part."""
    legal = masks.to(torch.float32)
    u = torch.rand(legal.shape[0], len(RADIX), generator=gen, device=legal.device)
    choices = []
    for k, (a, b) in enumerate(PARTS):
        cdf = legal[:, a:b].cumsum(1)
        target = u[:, k:k + 1] * cdf[:, -1:]
        choices.append((cdf <= target).sum(1).clamp_(max=b - a - 1))
    return pack(choices)
