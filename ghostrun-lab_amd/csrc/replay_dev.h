// The frame log replayed through FCEUmm's line renderer, wave-uniform (gfx950).
//
// The emulator kernels log every PPU-visible write of a frame with the dot its instruction starts at and its cycles
// (nes_dev.h log_event). Drawing a frame, finding its sprite-0 hit and resolving MMC2's latches all replay that log
// line by line the way the reference's NeSLE extension does (kdcyberdude/ghostrun-lab
// third_party/nesle-extensions.patch:1243-1812): a line's 34 tile slots are drawn in runs, each run up to the
// position where the next write lands (its instruction's end on FCEUmm's grid, 16 dots of lead-in before the line),
// with the state of that moment; Fixit1 (the vertical step) and Fixit2 (the horizontal copy) at their positions; the
// next line's sprites fetched after the pixels and latched at RefreshSprites.
//
// The walker below is the scalar part: the replay state is wave-uniform (SGPRs), events are read one at a time, and v
// moves over a run of slots in closed form. What a run draws is the sink's business:
//   - RenderSink (rlenv_hip.hip k_render): the 64 lanes fetch the run's tiles and shift out its pixels into a line
//     buffer in LDS, then compose sprites and write the observation row;
//   - S0Sink (here): the sprite-0 check of the emulator, which needs the background's opacity at 8 pixels of sprite
//     0's lines only; tiles are fetched lazily from descriptors of the slots, lines without writes are skipped in
//     closed form;
//   - LatchSink (here): MMC2's latch resolve, which needs no pixels at all.
// MMC2's latch hook after every pattern fetch is run by the walker itself, the fetches of a run of slots (or of a
// sprite line) on the lanes of the wavefront at once, so the sinks only receive the CHR pages each fetch read through.
// That part needs every lane active: the renderer's waves are, and an MMC2 console's emulation runs on all 64 lanes
// (emu_kernel.h emu_body).
#pragma once
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <stdint.h>
#endif

#include "nesrec.h"

namespace nd {

constexpr int32_t kNoCheck = 0x100;
constexpr int32_t kNoEvent = 0x7FFFFFFF;

__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ uint64_t uni64(uint64_t v) {
    return (uint64_t)uni((uint32_t)v) | ((uint64_t)uni((uint32_t)(v >> 32)) << 32);
}

// Replay time of NeSLE frame dot `dot` (patch:950-956): line 0 dot 0 is 0, the pre-render line is negative (a kook
// frame's one dot closer), and every time sits NES_FCEU_LAG dots after the NeSLE dot.
__device__ __forceinline__ int32_t fceu_time(uint32_t dot, uint32_t kook) {
    return dot >= NES_PRERENDER_DOT ? (int32_t)dot - (int32_t)NES_FRAME_DOTS + NES_FCEU_LAG + (int32_t)kook
                                    : (int32_t)dot + NES_FCEU_LAG;
}

// v after n one-tile steps to the right (FCEUmm's per-slot increment, the horizontal nametable flipping at each wrap).
__device__ __forceinline__ uint32_t v_steps(uint32_t v, uint32_t n) {
    const uint32_t cx = (v & 31u) + n;
    return (v & ~0x41Fu) | (cx & 31u) | ((((v >> 10) ^ (cx >> 5)) & 1u) << 10);
}

// v one pixel row down (Fixit1; patch:1410-1422): fine y, then the coarse row, which leaves row 29 for row 0 of the
// other vertical nametable and row 31 for row 0 of the same one.
__device__ __forceinline__ uint32_t y_step(uint32_t v) {
    if ((v & 0x7000u) != 0x7000u) return (v + 0x1000u) & 0x7FFFu;
    v &= ~0x7000u;
    const uint32_t row = (v >> 5) & 31u;
    if (row == 29u) return (v & ~0x03E0u) ^ 0x0800u;
    if (row == 31u) return v & ~0x03E0u;
    return v + 0x20u;
}

// y_step applied n times, in closed form: the pixel row (coarse * 8 + fine) counts up to 240, where it wraps to 0 of
// the other nametable, or from rows 240-255 (coarse 30, 31) up to 256, where it wraps without the flip.
__device__ __forceinline__ uint32_t y_steps(uint32_t v, uint32_t n) {
    uint32_t y = ((v >> 5) & 31u) * 8u + ((v >> 12) & 7u), nt = (v >> 11) & 1u;
    while (n) {
        const uint32_t wrap = y < 240u ? 240u : 256u, d = wrap - y;
        if (n < d) {
            y += n;
            break;
        }
        n -= d;
        if (wrap == 240u) nt ^= 1u;
        y = 0;
    }
    return (v & 0x041Fu) | ((y >> 3) << 5) | ((y & 7u) << 12) | (nt << 11);
}

__device__ __forceinline__ uint32_t nt_slot(uint32_t nt_map, uint32_t addr) {
    return ((nt_map >> (((addr >> 10) & 3u) * 2u)) & 1u) * 1024u + (addr & 0x3FFu);
}

// MMC2: an address in $0FD0-$0FEF / $1FD0-$1FEF flips the latch of its half (FCEUmm's PPU_hook ranges,
// patch:3196-3220, 1390-1402). 0 = none, else the latch value + 1 | half << 2.
__device__ __forceinline__ uint32_t mmc2_trigger(uint32_t a) {
    const uint32_t high = (a >> 8) & 0x3Fu, low = a & 0xF0u;
    if (high >= 0x20u || (high & 0x0Fu) != 0x0Fu || (low != 0xD0u && low != 0xE0u)) return 0;
    return (low == 0xE0u ? 2u : 1u) | (high < 0x10u ? 0u : 4u);
}

// The replay's state between lines (patch:1289-1313), wave-uniform. Sprite lines themselves belong to the sink; the
// walker keeps what RefreshSprites needs of the last fetch (the count, whether sprite 0 is in it, its first sprite).
struct Rs {
    uint32_t v, t, fx, ctrl, mask;
    uint32_t chr_lo, chr_hi;   // 1 KB CHR page of slots 0-3 / 4-7, 8 bits each
    uint32_t nt_map;
    uint32_t creg, latch;      // MMC2: the 4 CHR registers (8 bits each), latch 0 | latch 1 << 8
    uint32_t mmc2_pages;       // MMC2: the cart's 1 KB CHR pages; 0 on other boards
    uint32_t cur, count, kook;
    int32_t next;              // replay time of event cur's instruction start, kNoEvent when none is left
    uint32_t f_n, f_blurp, f_bits, f_attr, f_x;   // last sprite fetch: count, sprite 0 in it, first sprite's row
    uint32_t spork, hit;
    int32_t sphitx, hit_x;
    uint32_t sphit_bits;
};

__device__ __forceinline__ bool rs_rendering(const Rs& s) { return (s.mask & 0x18u) != 0; }
__device__ __forceinline__ uint32_t rs_inc(const Rs& s) { return (s.ctrl & 4u) ? 32u : 1u; }

template <class K>
__device__ __forceinline__ void rs_next(Rs& s, K& k) {
    s.next = s.cur < s.count ? fceu_time((k.ev(2u * s.cur) >> 8) & 0x1FFFFu, s.kook) : kNoEvent;
}

// MMC2: half `half`'s slots from its register and latch (patch:1385-1388).
__device__ __forceinline__ void rs_mmc2_select(Rs& s, uint32_t half) {
    const uint32_t reg = 2u * half + ((s.latch >> (8u * half)) & 1u);
    const uint32_t bank = (s.creg >> (8u * reg)) & 0xFFu;
    uint32_t pk = 0;
    for (uint32_t i = 0; i < 4u; ++i) pk |= ((bank * 4u + i) & (s.mmc2_pages - 1u)) << (8u * i);
    if (half) s.chr_hi = pk;
    else s.chr_lo = pk;
}
// This lane's index in the wavefront.
__device__ __forceinline__ uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// MMC2: a run of pattern fetches, one per lane in fetch order (lane order, `mine` on the lanes that fetch, at pa),
// with every lane of the wavefront active. Each fetch reads through its half's pages as the hooks of the fetches
// before it left them, then flips its half's latch if pa is a trigger (FCEUmm's PPU_hook after the fetch,
// patch:1390-1402): the page it read through is returned on its lane, and the latches and pages after the whole run
// are left in s. The same as hooking one fetch at a time: a fetch's pattern address does not depend on the latches.
__device__ inline uint32_t rs_mmc2_fetches(Rs& s, bool mine, uint32_t pa) {
    const uint32_t t = mine ? mmc2_trigger(pa) : 0u, half = (pa >> 12) & 1u;
    const uint64_t t0 = __ballot(t != 0u && (t & 4u) == 0u), t1 = __ballot((t & 4u) != 0u);
    const uint64_t fe = __ballot((t & 3u) == 2u);   // triggers that set their latch to 1 ($xFE0-$xFEF)
    const uint64_t before = (half ? t1 : t0) & (((uint64_t)1 << lane_id()) - 1u);
    uint32_t pk = half ? s.chr_hi : s.chr_lo;
    if (before) {   // the last trigger of this half before this fetch set the latch
        const uint32_t bit = (uint32_t)(fe >> (63 - __builtin_clzll(before))) & 1u;
        const uint32_t bank = (s.creg >> (8u * (2u * half + bit))) & 0xFFu;
        pk = 0;
        for (uint32_t i = 0; i < 4u; ++i) pk |= ((bank * 4u + i) & (s.mmc2_pages - 1u)) << (8u * i);
    }
    for (uint32_t h = 0; h < 2u; ++h) {
        const uint64_t th = h ? t1 : t0;
        if (!th) continue;
        const uint32_t bit = (uint32_t)(fe >> (63 - __builtin_clzll(th))) & 1u;
        s.latch = (s.latch & ~(0xFFu << (8u * h))) | (bit << (8u * h));
        rs_mmc2_select(s, h);
    }
    return pk;
}

// The replay from the log header (patch:1361-1383): `log` = header + events (global memory), `n` events (read through
// the sink).
template <class K>
__device__ inline void rs_load(Rs& s, K& k, const uint32_t* log, uint32_t n, uint32_t mmc2_pages) {
    const uint32_t h1 = uni(log[1]), h2 = uni(log[2]), h5 = uni(log[5]);
    s.ctrl = h1 & 0xFFu;
    s.mask = (h1 >> 8) & 0xFFu;
    s.fx = (h1 >> 16) & 7u;
    s.v = h2 & 0x7FFFu;
    s.t = (h2 >> 16) & 0x7FFFu;
    s.chr_lo = uni(log[3]);
    s.chr_hi = uni(log[4]);
    s.nt_map = h5 & 0xFFu;
    s.kook = (h5 & NES_LOG_KOOK) ? 1u : 0u;
    s.creg = uni(log[14]);
    s.latch = uni(log[15]);
    s.mmc2_pages = mmc2_pages;
    s.count = n < NES_LOG_EVENTS ? n : NES_LOG_EVENTS;
    s.cur = 0;
    s.f_n = s.f_blurp = s.f_bits = s.f_attr = s.f_x = 0;
    s.spork = s.hit = 0;
    s.sphitx = kNoCheck;
    s.hit_x = -1;
    s.sphit_bits = 0;
    rs_next(s, k);
}

// Event cur applied to the replay (patch:1424-1481); palette writes go to the sink. `drawing`: a line is drawn.
template <class K>
__device__ inline void rs_apply(Rs& s, K& k, bool drawing) {
    const uint32_t w0 = k.ev(2u * s.cur), w1 = k.ev(2u * s.cur + 1u);
    const uint32_t kind = w0 & 15u, val = w1 & 0xFFu, aux = (w1 >> 8) & 0xFFu;
    ++s.cur;
    rs_next(s, k);
    if (kind == NES_EV_CTRL) {
        s.ctrl = val;
        s.t = (s.t & 0xF3FFu) | ((val & 3u) << 10);
    } else if (kind == NES_EV_MASK) {
        s.mask = val;
    } else if (kind == NES_EV_SCROLL) {
        if (aux == 0) {
            s.t = (s.t & 0xFFE0u) | (val >> 3);
            s.fx = val & 7u;
        } else {
            s.t = (s.t & 0x0C1Fu) | ((val & 7u) << 12) | ((val & 0xF8u) << 2);
        }
    } else if (kind == NES_EV_ADDR) {
        if (aux == 0) {
            s.t = (s.t & 0x00FFu) | ((val & 0x3Fu) << 8);
        } else {
            s.t = (s.t & 0xFF00u) | val;
            s.v = s.t;
        }
    } else if (kind == NES_EV_DATA) {
        s.v = (s.v + (aux + 1u) * rs_inc(s)) & 0x7FFFu;
    } else if (kind == NES_EV_DREAD) {
        s.v = drawing && rs_rendering(s) ? y_step(s.v) : ((s.v + rs_inc(s)) & 0x7FFFu);
    } else if (kind == NES_EV_PAL) {
        k.palette(aux & 31u, val);
        s.v = (s.v + rs_inc(s)) & 0x7FFFu;
    } else if (kind == NES_EV_CHR) {
        const uint32_t sh = (aux & 3u) * 8u, keep = ~(0xFFu << sh);
        if (aux & 4u) s.chr_hi = (s.chr_hi & keep) | (val << sh);
        else s.chr_lo = (s.chr_lo & keep) | (val << sh);
    } else if (kind == NES_EV_MIRROR) {
        s.nt_map = val;
    } else if (kind == NES_EV_MMC2) {
        if (aux < 4u) {
            s.creg = (s.creg & ~(0xFFu << (8u * aux))) | (val << (8u * aux));
            rs_mmc2_select(s, aux >> 1);
        } else if (aux == 6u || aux == 7u) {
            const uint32_t h = aux - 6u;
            s.latch = (s.latch & ~(0xFFu << (8u * h))) | ((val & 1u) << (8u * h));
            rs_mmc2_select(s, h);
        }
    }
}

template <class K>
__device__ __forceinline__ void rs_apply_before(Rs& s, K& k, int32_t time, bool drawing) {
    while (s.next < time) rs_apply(s, k, drawing);
}

// The pre-render line: the writes before line 0's lead-in, then v = t while rendering (patch:1483-1490).
template <class K>
__device__ inline void rs_begin_frame(Rs& s, K& k) {
    rs_apply_before(s, k, -NES_LINE_LEAD, false);
    if (rs_rendering(s)) s.v = s.t;
}

// One line being drawn: the next tile slot, the output position, the vertical step still due.
struct Ln {
    int32_t tile, out;
    bool fix;
};

// Tile slots [ln.tile, last) with the state as it is (FCEUmm's tile loop, patch:1496-1577): with rendering off the
// backdrop, advancing the output position for every slot, the two prefetch slots included; else the sink fetches
// and shifts them out. MMC2: each fetch reads through the pages of the moment and then flips its latch.
template <class K>
__device__ inline void rs_tiles(Rs& s, K& k, Ln& ln, int32_t last, bool pixels) {
    const int32_t first = ln.tile;
    if (!rs_rendering(s)) {
        k.off_run(ln.out, 8 * (last - first), pixels);
        ln.out += 8 * (last - first);
        ln.tile = last;
        return;
    }
    if (s.mmc2_pages) {   // lane j fetches slot j
        const int32_t j = (int32_t)lane_id();
        const bool mine = j >= first && j < last;
        uint32_t pa = 0;
        if (mine) {
            const uint32_t v = v_steps(s.v, (uint32_t)(j - first));
            pa = k.nt_lane(nt_slot(s.nt_map, 0x2000u | (v & 0x0FFFu))) * 16u + ((s.ctrl & 0x10u) << 8) + ((v >> 12) & 7u);
        }
        const uint32_t pk = rs_mmc2_fetches(s, mine, pa);
        if (mine) k.slot_pages(j, pk);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // the pages, read by other lanes
    }
    k.on_run(s, first, last, ln.out, pixels);
    s.v = v_steps(s.v, (uint32_t)(last - first));
    const int32_t from = first > 2 ? first : 2;
    if (last > from) ln.out += 8 * (last - from);
    ln.tile = last;
}

// The sprite-0 check against the background drawn left of position p - 16 (patch:1583-1594).
template <class K>
__device__ __forceinline__ void rs_check(Rs& s, K& k, int32_t p) {
    if (s.sphitx == kNoCheck) return;
    int32_t end = s.sphitx + 8;
    if (end > p - 16) end = p - 16;
    if (end > 255) end = 255;
    if (end <= s.sphitx) return;
    const int32_t x = k.find_hit(s.sphitx, s.sphit_bits, end);
    if (x >= 0) {
        s.hit = 1;
        s.hit_x = x;
        s.sphitx = kNoCheck;
    }
}

// The line drawn up to position p (RefreshLine for an access there, patch:1596-1613).
template <class K>
__device__ inline void rs_update(Rs& s, K& k, Ln& ln, int32_t p, bool pixels) {
    int32_t last = p >> 3;
    if (pixels && s.sphitx != kNoCheck && s.sphitx < p - 16 && s.sphitx >= (last - 2) * 8) ++last;
    if (last > 34) last = 34;
    if (last <= ln.tile) return;
    rs_tiles(s, k, ln, last, pixels);
    if (p >= 268 && ln.fix) {
        if (rs_rendering(s)) s.v = y_step(s.v);
        ln.fix = false;
    }
    if (pixels) rs_check(s, k, p);
}

// Line l: its pixels with every write that lands while it is drawn, at its instruction's end; $2007 writes draw
// nothing first (patch:1617-1634).
template <class K>
__device__ inline void rs_line(Rs& s, K& k, int32_t l, bool pixels) {
    const int32_t start = l * 341 - NES_LINE_LEAD;
    Ln ln{0, 0, true};
    k.line_begin(s, pixels);
    while (s.next < start + 272) {
        const uint32_t w0 = k.ev(2u * s.cur), kind = w0 & 15u;
        if (kind != NES_EV_DATA && kind != NES_EV_PAL) rs_update(s, k, ln, s.next + 3 * (int32_t)((w0 >> 4) & 15u) - start, pixels);
        rs_apply(s, k, true);
    }
    rs_update(s, k, ln, 272, pixels);
    if (ln.fix && rs_rendering(s)) s.v = y_step(s.v);
    if (pixels) rs_check(s, k, 272);
}

// Sprite-line fetch for line l + 1 (FetchSpriteData, patch:1671-1700): the sink fetches; MMC2's hooks run here in
// OAM order, lane i = OAM entry i, the first eight entries on the line fetching (the sink gets each fetch's pages
// through sprite_pages, on the lane of the entry, by its rank).
template <class K>
__device__ inline void rs_fetch_sprites(Rs& s, K& k, int32_t l) {
    if (s.mmc2_pages) {
        const uint32_t ctrl = s.ctrl, h = (ctrl & 0x20u) ? 16u : 8u;
        const uint32_t table8 = (ctrl & 0x08u) && !(ctrl & 0x20u) ? 0x1000u : 0u;
        const uint32_t e = k.oam_lane(lane_id());   // y, tile, attribute, x
        const uint32_t row = (uint32_t)(l - (int32_t)(e & 0xFFu));
        const uint64_t on = __ballot(row < h);
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(on >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)on, 0u));
        const bool mine = row < h && rank < 8u;
        uint32_t pa = 0;
        if (mine) {
            const uint32_t tile = (e >> 8) & 0xFFu, attr = (e >> 16) & 0xFFu;
            pa = h == 16u ? ((tile & 1u) << 12) + ((tile & 0xFEu) << 4) : (tile << 4) + table8;
            if (attr & 0x80u) pa += 7u - row + ((ctrl & 0x20u) >> 1) - (row & 8u);
            else pa += row + (row & 8u);
            pa &= 0x1FFFu;
        }
        const uint32_t pk = rs_mmc2_fetches(s, mine, pa);
        if (mine) k.sprite_pages(rank, pk);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    k.fetch_sprites(s, l);
}

// After line l's pixels (patch:1666-1730): the next line's sprites, the writes before the horizontal copy (grid dot
// 262), Fixit2, the writes up to the line's end, and RefreshSprites with sprites on: the fetched line becomes the one
// drawn next, with the sprite palette of the moment and sprite 0's check when it is in the line and not hit yet.
template <class K>
__device__ inline void rs_end_of_line(Rs& s, K& k, int32_t l, bool sprites) {
    const int32_t start = l * 341 - NES_LINE_LEAD;
    s.sphitx = kNoCheck;
    if (rs_rendering(s) && (sprites || s.mmc2_pages)) rs_fetch_sprites(s, k, l);
    rs_apply_before(s, k, start + 278, true);
    if (rs_rendering(s)) s.v = (s.v & 0xFBE0u) | (s.t & 0x041Fu);
    rs_apply_before(s, k, start + 341, true);
    if (s.mask & 0x10u) {
        s.spork = 0;
        if (s.f_n != 0) {
            k.latch_sprites(s);
            if (s.f_blurp && !s.hit && s.f_bits) {
                uint32_t b = s.f_bits;
                if (s.f_attr & 0x40u) b = __builtin_bitreverse32(b) >> 24;
                s.sphitx = (int32_t)s.f_x;
                s.sphit_bits = b;
            }
            s.spork = 1;
        }
    }
}

// CHR byte through packed slot pages (lo: slots 0-3, hi: slots 4-7).
__device__ __forceinline__ uint32_t chr_pk(const uint8_t* chr_rom, const uint8_t* chr_ram, uint32_t lo, uint32_t hi,
                                          uint32_t a) {
    const uint32_t slot = (a >> 10) & 7u;
    const uint32_t page = ((slot & 4u ? hi : lo) >> ((slot & 3u) * 8u)) & 0xFFu;
    const uint32_t off = page * 1024u + (a & 0x3FFu);
    return chr_rom ? chr_rom[off] : chr_ram[off & (NES_CHRRAM_BYTES - 1u)];
}

// ------------------------------------------------------------------------------------------ sprite 0
// What the emulator's sprite-0 check needs: the background's opacity under sprite 0's 8 pixels on its lines. A slot's
// fetch is kept as a descriptor (v | pattern table << 15 | nametable map << 16, and the slot pages) and fetched only
// when its pixels fall under sprite 0.
struct S0Sink {
    const uint32_t* ev_mem;      // the log's events (global memory, written by this kernel)
    const uint8_t* nt_mem;       // the console's nametables and OAM as they are now (LDS)
    const uint8_t* oam_mem;
    const uint8_t *chr_rom, *chr_ram;
    uint32_t d0, d0lo, d0hi;     // descriptors of the last two slots fetched (d1 the latest)
    uint32_t d1, d1lo, d1hi;
    uint32_t* pages;             // MMC2: the pages each slot of the run read through (34 words of LDS)
    uint32_t opq;                // sprite 0's 8 pixels on this line: bit i set = pixel sphitx + i opaque background
    int32_t x0;                  // sphitx of this line (kNoCheck: no check, nothing to track)

    __device__ uint32_t ev(uint32_t i) { return uni(ev_mem[i]); }
    __device__ uint32_t nt(uint32_t i) { return uni(nt_mem[i]); }
    __device__ uint32_t oam(uint32_t i) { return uni(oam_mem[i]); }
    __device__ uint32_t nt_lane(uint32_t i) { return nt_mem[i]; }
    __device__ uint32_t oam_lane(uint32_t i) { return reinterpret_cast<const uint32_t*>(oam_mem)[i]; }
    __device__ void palette(uint32_t, uint32_t) {}
    __device__ uint32_t page(int32_t j) { return uni(pages[j]); }
    // (MMC2 pages: written on the lane of the fetch)
    __device__ void slot_pages(int32_t j, uint32_t pk) { pages[j] = pk; }
    __device__ void sprite_pages(uint32_t n, uint32_t pk) {
        if (n == 0) pages[0] = pk;   // (the run's pages are done with by the time sprites are fetched)
    }
    __device__ void line_begin(const Rs& s, bool pixels) {
        x0 = pixels ? s.sphitx : kNoCheck;
        opq = 0;
    }
    // pattern bytes (lo | hi << 8) of a descriptor
    __device__ uint32_t fetch(uint32_t d, uint32_t lo, uint32_t hi) {
        const uint32_t v = d & 0x7FFFu;
        const uint32_t pa = nt(nt_slot(d >> 16, 0x2000u | (v & 0x0FFFu))) * 16u + ((d >> 15) & 1u) * 0x1000u +
                            ((v >> 12) & 7u);
        return uni(chr_pk(chr_rom, chr_ram, lo, hi, pa)) | (uni(chr_pk(chr_rom, chr_ram, lo, hi, pa + 8u)) << 8);
    }
    // Pixels [o, o + n) of the line drawn transparent (backdrop or hidden) as far as they fall under sprite 0.
    __device__ void clear(int32_t o, int32_t n) {
        if (x0 == kNoCheck) return;
        for (int32_t i = 0; i < 8; ++i)
            if (x0 + i >= o && x0 + i < o + n) opq &= ~(1u << i);
    }
    __device__ void off_run(int32_t out, int32_t n, bool pixels) {
        if (pixels) clear(out, n);
    }
    __device__ void on_run(const Rs& s, int32_t first, int32_t last, int32_t out, bool pixels) {
        const uint32_t base = ((s.ctrl & 0x10u) << 11) | (s.nt_map << 16);
        const bool mmc2 = s.mmc2_pages != 0;
        if (pixels && x0 != kNoCheck) {
            // the slots whose 8 output pixels meet sprite 0's: slot k >= from writes pixels out + 8 (k - from)
            const int32_t from = first > 2 ? first : 2;
            for (int32_t k = from; k < last; ++k) {
                const int32_t o = out + 8 * (k - from);
                if (o >= 256 || o + 8 <= x0 || o >= x0 + 8) continue;
                // the two fetches before slot k: of this run, or carried from before it
                uint32_t a, alo, ahi, b, blo, bhi;
                auto desc = [&](int32_t j, uint32_t& d, uint32_t& lo, uint32_t& hi) {
                    d = v_steps(s.v, (uint32_t)(j - first)) | base;
                    lo = mmc2 ? page(j) : s.chr_lo;
                    hi = mmc2 ? page(j) : s.chr_hi;
                };
                if (k - first >= 2) {
                    desc(k - 2, a, alo, ahi);
                    desc(k - 1, b, blo, bhi);
                } else if (k - first == 1) {
                    a = d1; alo = d1lo; ahi = d1hi;
                    desc(k - 1, b, blo, bhi);
                } else {
                    a = d0; alo = d0lo; ahi = d0hi;
                    b = d1; blo = d1lo; bhi = d1hi;
                }
                const uint32_t pa = fetch(a, alo, ahi), pb = fetch(b, blo, bhi);
                const uint32_t lo16 = ((pa & 0xFFu) << 8) | (pb & 0xFFu), hi16 = (pa & 0xFF00u) | (pb >> 8);
                for (int32_t q = 0; q < 8; ++q) {
                    const int32_t i = o + q - x0;
                    if (i < 0 || i >= 8) continue;
                    const uint32_t bit = 15u - s.fx - (uint32_t)q;
                    if (((lo16 | hi16) >> bit) & 1u) opq |= 1u << i;
                    else opq &= ~(1u << i);
                }
            }
            if (first <= 2 && last > 2 && !(s.mask & 0x02u)) clear(0, 8);
            if (!(s.mask & 0x08u)) {
                int32_t f = first - 2, n = last - first;
                if (f < 0) {
                    n += f;
                    f = 0;
                }
                clear(8 * f, 8 * n);
            }
        }
        // the run's last two fetches are the ones the next run starts from
        if (last - first >= 2) {
            uint32_t lo, hi;
            d0 = v_steps(s.v, (uint32_t)(last - 2 - first)) | base;
            d0lo = mmc2 ? page(last - 2) : s.chr_lo;
            d0hi = mmc2 ? page(last - 2) : s.chr_hi;
            d1 = v_steps(s.v, (uint32_t)(last - 1 - first)) | base;
            lo = mmc2 ? page(last - 1) : s.chr_lo;
            hi = mmc2 ? page(last - 1) : s.chr_hi;
            d1lo = lo;
            d1hi = hi;
        } else {
            d0 = d1; d0lo = d1lo; d0hi = d1hi;
            d1 = s.v | base;
            d1lo = mmc2 ? page(first) : s.chr_lo;
            d1hi = mmc2 ? page(first) : s.chr_hi;
        }
    }
    // (bits: sprite 0's opaque pixels, leftmost in bit 7; opq: leftmost in bit 0)
    __device__ int32_t find_hit(int32_t x, uint32_t bits, int32_t end) {
        const uint32_t m = opq & (__builtin_bitreverse32(bits) >> 24) & ((1u << (end - x)) - 1u);
        return m ? x + (int32_t)__builtin_ctz(m) : -1;
    }
    // Sprite 0's row when it is in the line (the sprite-0 setup needs only that: a fetched line without sprite 0
    // sets no check).
    __device__ void fetch_sprites(Rs& s, int32_t l) {
        const uint32_t ctrl = s.ctrl, h = (ctrl & 0x20u) ? 16u : 8u;
        const uint32_t y = oam(0u), row = (uint32_t)(l - (int32_t)y);
        s.f_blurp = row < h ? 1u : 0u;
        s.f_n = s.f_blurp;
        if (!s.f_blurp) return;
        const uint32_t tile = oam(1u), attr = oam(2u);
        const uint32_t table8 = (ctrl & 0x08u) && !(ctrl & 0x20u) ? 0x1000u : 0u;
        uint32_t pa = h == 16u ? ((tile & 1u) << 12) + ((tile & 0xFEu) << 4) : (tile << 4) + table8;
        if (attr & 0x80u) pa += 7u - row + ((ctrl & 0x20u) >> 1) - (row & 8u);
        else pa += row + (row & 8u);
        pa &= 0x1FFFu;
        const uint32_t lo = s.mmc2_pages ? page(0) : s.chr_lo, hi = s.mmc2_pages ? page(0) : s.chr_hi;
        s.f_bits = uni(chr_pk(chr_rom, chr_ram, lo, hi, pa)) | uni(chr_pk(chr_rom, chr_ram, lo, hi, pa + 8u));
        s.f_attr = attr;
        s.f_x = oam(3u);
    }
    __device__ void latch_sprites(const Rs&) {}
};

// The frame's sprite-0 hit from the log so far (NeSLE's frame_sprite0_hit, patch:1752-1788), over the console's
// nametables and OAM as they are now: the NeSLE frame dot from which an instruction sees the flag (*hit = true), or,
// with no hit, the dot after which no write can make one (the end of sprite 0's lines), or 0 when sprite 0 is below
// the picture. Lines before sprite 0's first one are replayed without pixels, runs of lines without writes in closed form. pages: 34 words of scratch LDS (MMC2).
__device__ __forceinline__ uint32_t sprite0_hit(const uint32_t* log, uint32_t log_n, const uint8_t* nt,
                                                const uint8_t* oam, const uint8_t* chr_rom, const uint8_t* chr_ram,
                                                uint32_t mmc2_pages, uint32_t* pages, uint32_t* hit_out) {
    *hit_out = 0;
    const int32_t first = (int32_t)uni(oam[0]) + 1;
    if (first >= 240) return 0;
    Rs s;
    S0Sink k;
    k.ev_mem = log + NES_LOG_HDR_WORDS;
    rs_load(s, k, log, log_n, mmc2_pages);
    k.nt_mem = nt;
    k.oam_mem = oam;
    k.chr_rom = chr_rom;
    k.chr_ram = chr_ram;
    k.pages = pages;
    k.d0 = k.d0lo = k.d0hi = k.d1 = k.d1lo = k.d1hi = 0;
    k.opq = 0;
    k.x0 = kNoCheck;
    rs_begin_frame(s, k);
    const int32_t last = first + 15 < 239 ? first + 15 : 239;
    for (int32_t l = 0; l <= last; ++l) {
        if (!s.mmc2_pages && l < first - 1) {
            // lines l .. l2 - 1 hold no write and fetch no sprites: Fixit1 and Fixit2 once a line while rendering,
            // the last line's slots 32 and 33 the latest fetches
            const int32_t stop = s.next >= (first - 1) * 341 - NES_LINE_LEAD ? first - 1 : (s.next + NES_LINE_LEAD) / 341;
            const int32_t n = stop - l;
            if (n >= 1) {
                if (rs_rendering(s)) {
                    const uint32_t base = ((s.ctrl & 0x10u) << 11) | (s.nt_map << 16);
                    const uint32_t vl = n >= 2 ? ((y_steps(s.v, (uint32_t)(n - 1)) & 0x7BE0u) | (s.t & 0x041Fu)) : s.v;
                    k.d0 = v_steps(vl, 32u) | base;
                    k.d1 = v_steps(vl, 33u) | base;
                    k.d0lo = k.d1lo = s.chr_lo;
                    k.d0hi = k.d1hi = s.chr_hi;
                    s.v = (y_steps(s.v, (uint32_t)n) & 0x7BE0u) | (s.t & 0x041Fu);
                }
                if (s.mask & 0x10u) s.spork = s.f_n != 0 ? 1u : 0u;
                s.sphitx = kNoCheck;
                l = stop - 1;
                continue;
            }
        }
        const int32_t sphitx = s.sphitx;
        rs_line(s, k, l, l >= first);
        if (s.hit) {
            // the first line position that has drawn pixel hit_x (patch:1743-1750), minus a 4-cycle read's 12 dots
            int32_t p = s.hit_x + 17;
            for (;; ++p) {
                int32_t lt = p >> 3;
                if (sphitx < p - 16 && sphitx >= (lt - 2) * 8) ++lt;
                if (lt > 34) lt = 34;
                if (s.hit_x < (lt - 2) * 8) break;
            }
            *hit_out = 1;
            return (uint32_t)(l * 341 - NES_LINE_LEAD + p - 12 - NES_FCEU_LAG);
        }
        s.spork = 0;
        rs_end_of_line(s, k, l, l >= first - 1);
    }
    return (uint32_t)(last * 341 + 256 - NES_FCEU_LAG);
}

// ------------------------------------------------------------------------------------------- MMC2
// The latches-only replay: every pattern fetch's hook runs in the walker, nothing is drawn.
struct LatchSink {
    const uint32_t* ev_mem;
    const uint8_t* nt_mem;
    const uint8_t* oam_mem;
    __device__ uint32_t ev(uint32_t i) { return uni(ev_mem[i]); }
    __device__ uint32_t nt(uint32_t i) { return uni(nt_mem[i]); }
    __device__ uint32_t oam(uint32_t i) { return uni(oam_mem[i]); }
    __device__ uint32_t nt_lane(uint32_t i) { return nt_mem[i]; }
    __device__ uint32_t oam_lane(uint32_t i) { return reinterpret_cast<const uint32_t*>(oam_mem)[i]; }
    __device__ void palette(uint32_t, uint32_t) {}
    __device__ void slot_pages(int32_t, uint32_t) {}
    __device__ void sprite_pages(uint32_t, uint32_t) {}
    __device__ void line_begin(const Rs&, bool) {}
    __device__ void off_run(int32_t, int32_t, bool) {}
    __device__ void on_run(const Rs&, int32_t, int32_t, int32_t, bool) {}
    __device__ int32_t find_hit(int32_t, uint32_t, int32_t) { return -1; }
    __device__ void fetch_sprites(Rs&, int32_t) {}
    __device__ void latch_sprites(const Rs&) {}
};

// MMC2 at vblank: the latches this frame's own pattern fetches leave (NeSLE's frame_resolve_mmc2, patch:1790-1812;
// the reference env runs it right after the vblank stop, rl/csrc/nes_machine.cuh:110-131). Returns latch 0 | latch 1
// << 8.
__device__ __forceinline__ uint32_t mmc2_latches(const uint32_t* log, uint32_t log_n, const uint8_t* nt, const uint8_t* oam,
                                              uint32_t chr_pages) {
    Rs s;
    LatchSink k{log + NES_LOG_HDR_WORDS, nt, oam};
    rs_load(s, k, log, log_n, chr_pages);
    rs_begin_frame(s, k);
    for (int32_t l = 0; l < 240; ++l) {
        rs_line(s, k, l, false);
        rs_end_of_line(s, k, l, true);
    }
    while (s.cur < s.count) rs_apply(s, k, false);
    return s.latch;
}

}  // namespace nd
