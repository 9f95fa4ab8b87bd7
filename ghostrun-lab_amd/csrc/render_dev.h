// The picture of one console-frame (gfx950): FCEUmm's line renderer over the frame log, the renderer's side of the
// line replay of replay_dev.h. Shared by the library's render kernel (rlenv_hip.hip k_render, which draws a frame the
// emulator kernel logged) and the console-frame kernel that emulates and then draws its own frame (emu_kernel.h
// emu_body with kDraw, also in the kernels compiled at run time from a cartridge's translated blocks).
#pragma once
#ifndef __HIPCC_RTC__   // (built in where hiprtc compiles this at run time)
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#include "nes_dev.h"
#include "replay_dev.h"
#include "rlenv_state.h"

namespace nd {

// The renderer's side of the line replay (replay_dev.h): the walker runs wave-uniform on every lane and hands each run
// of tile slots here, where the 64 lanes work on it in LDS:
//   - fetch: lane j fetches slot j's tile (nametable tile and attribute, both pattern bytes) into F[j + 2];
//   - output: lane k >= 2 shifts out slot k's 8 pixels - the two fetches before it, fine x, the palette of the moment -
//     into the line buffer at the run's output position (F[0], F[1] carry the line's first fetches' predecessors);
//   - the run's hidden left column and background-off range, then the sprite-0 check over 8 lanes.
// Sprite lines are fetched with one ballot over the 64 OAM entries (lane = sprite) into one of two buffers; the one
// RefreshSprites latched is expanded at the start of the line it is drawn on (lane 8k + p = pixel p of sprite k) into
// a sprite line with one LDS max per pixel, which picks the lowest-numbered opaque sprite.
// A run of lines with no write (most of them) takes fast_run: per line one fetch phase, one sync, and each lane
// composes its 4 pixels in registers.
// The render's LDS besides the nametables and OAM (1,720 bytes; the console-frame kernel that draws its own frame lays
// it over the CPU RAM it has copied out).
struct RenderScratch {
    uint32_t px[64];          // the line: palette value, 0x40 | backdrop where the background is transparent (in
                              // fast_run, which draws in registers: where the lanes that fetch no sprite store)
    uint32_t sp[256];         // the sprite line: (7 - rank) << 8 | behind << 7 | palette << 2 | value, 0 = none
    uint32_t f[36];           // fetches: lo | hi << 8 | attribute << 16; 0-1 carried, 2 + j slot j
    uint32_t spr[2][8];       // sprite lines: lo | hi << 8 | attr << 16 | x << 24
    uint32_t pages[34 + 8];   // MMC2: the pages of each slot's fetch, then of each sprite's
    uint4 tab[2];             // the background palette table (bg_table), the latched sprite palette (latch_sprites)
    alignas(16) uint8_t pal[32];
};

typedef __attribute__((address_space(4))) const uint32_t KU32;

// kScalarLog: the frame log was written before this kernel, so its events are read through the scalar cache; else
// (written earlier in this kernel, by lane 0) by vector loads after the workgroup sync.
template <bool kScalarLog>
struct RenderSink {
    RenderScratch* L;
    uint8_t *ntab, *otab;     // the console's nametables and OAM as of the frame's vblank stop (LDS)
    const uint32_t* log;      // the console's frame log
    const uint8_t *chr_rom, *chr_ram;
    const uint16_t* chr_pairs;   // CHR ROM by tile row (both planes in one word), nullptr with CHR RAM
    int lane;
    bool mmc2;
    uint32_t ha, hb;          // F indices of the last two fetches
    uint32_t fetched, drawn, drawn_n;
    // L->tab[0] and L->tab[1] are rebuilt only after a palette write
    bool bg_stale, sp_stale;

    __device__ uint32_t ev(uint32_t i) {
        if constexpr (kScalarLog) return ((KU32*)(log + NES_LOG_HDR_WORDS))[i];
        else return uni(log[NES_LOG_HDR_WORDS + i]);
    }
    __device__ uint32_t nt(uint32_t i) { return uni(ntab[i]); }
    __device__ uint32_t oam(uint32_t i) { return uni(otab[i]); }
    __device__ uint32_t nt_lane(uint32_t i) { return ntab[i]; }
    __device__ uint32_t oam_lane(uint32_t i) { return reinterpret_cast<const uint32_t*>(otab)[i]; }
    __device__ uint32_t back() { return ((uint32_t)L->pal[0] & 0x3Fu) | 0x40u; }
    __device__ void palette(uint32_t i, uint32_t v) {
        if (lane == 0) L->pal[i] = (uint8_t)v;
        __syncthreads();
        bg_stale = sp_stale = true;
    }
    // MMC2: the pages of slot j's fetch, of the fetch of the line's sprite n (on the lane of the fetch)
    __device__ void slot_pages(int32_t j, uint32_t pk) { L->pages[j] = pk; }
    __device__ void sprite_pages(uint32_t n, uint32_t pk) { L->pages[34 + n] = pk; }
    // The latched sprite line expanded into L->sp (before the line's first sync; the compose reads and clears it).
    __device__ void expand_sprites(const Rs& s) {
        if (!s.spork) return;
        const uint32_t k = (uint32_t)lane >> 3, p = (uint32_t)lane & 7u;
        if (k < drawn_n) {
            const uint32_t e = L->spr[drawn][k];
            const uint32_t attr = (e >> 16) & 0xFFu, b = (attr & 0x40u) ? p : 7u - p;
            const uint32_t val = ((e >> b) & 1u) | (((e >> (8u + b)) & 1u) << 1);
            const uint32_t x = (e >> 24) + p;
            if (val && x < 256u)
                atomicMax(&L->sp[x], ((7u - k) << 8) | ((attr & 0x20u) << 2) | ((attr & 3u) << 2) | val);
        }
    }
    // A new line (general path): the last two fetches move to F[0], F[1]; nothing drawn yet (0xFF reads as
    // transparent); the sprite line expanded.
    __device__ void line_begin(const Rs& s, bool) {
        const uint32_t carry = lane < 2 ? L->f[lane ? hb : ha] : 0u;
        __syncthreads();
        if (lane < 2) L->f[lane] = carry;
        L->px[lane] = 0xFFFFFFFFu;
        ha = 0;
        hb = 1;
        expand_sprites(s);
        __syncthreads();
    }
    // Pixels [o, o + n) the backdrop (o and n multiples of 8).
    __device__ void fill(int32_t o, int32_t n) {
        const int32_t x = 4 * lane;
        if (x >= o && x < o + n) L->px[lane] = back() * 0x01010101u;
    }
    __device__ void off_run(int32_t out, int32_t n, bool) {
        fill(out, n);
        __syncthreads();
    }
    // The two plane bytes of pattern address pa (a row of plane 0; pa + 8 is plane 1) through the packed pages,
    // plane 0 in the low byte: one 16-bit load with CHR ROM (kPairs), two byte loads with CHR RAM.
    template <bool kPairs>
    __device__ uint32_t pattern_of(uint32_t lo, uint32_t hi, uint32_t pa) {
        if constexpr (!kPairs) {
            return chr_pk(chr_rom, chr_ram, lo, hi, pa) | (chr_pk(chr_rom, chr_ram, lo, hi, pa + 8u) << 8);
        } else {
            // the 1 KB slot's page: byte (pa >> 10) & 7 of hi:lo, one byte permute
            const uint32_t page = __builtin_amdgcn_perm(hi, lo, (pa >> 10) & 7u) & 0xFFu;
            return chr_pairs[page * 512u + ((pa & 0x3F0u) >> 1) + (pa & 7u)];
        }
    }
    // The chr_pairs index of pattern address pa (kPairs): its 1 KB page's, the tile's 8 rows, the row.
    __device__ uint32_t pairs_index(uint32_t lo, uint32_t hi, uint32_t pa) {
        const uint32_t page = __builtin_amdgcn_perm(hi, lo, (pa >> 10) & 7u) & 0xFFu;
        return page * 512u + ((pa & 0x3F0u) >> 1) + (pa & 7u);
    }
    __device__ uint32_t pattern(uint32_t lo, uint32_t hi, uint32_t pa) {
        return chr_pairs ? pattern_of<true>(lo, hi, pa) : pattern_of<false>(lo, hi, pa);
    }
    // Slot j's tile (nametable tile and attribute, both pattern bytes) fetched at v into F[j + 2].
    __device__ void fetch_slot(const Rs& s, uint32_t v, uint32_t j, uint32_t lo, uint32_t hi) {
        const uint32_t ntb = 0x2000u | (v & 0x0C00u), col = v & 31u;
        const uint32_t tile = ntab[nt_slot(s.nt_map, ntb | (v & 0x3FFu))];
        const uint32_t at = ntab[nt_slot(s.nt_map, ntb | 0x3C0u | (col >> 2) | ((v & 0x380u) >> 4))];
        const uint32_t sel = (at >> ((col & 2u) | ((v & 0x40u) >> 4))) & 3u;
        const uint32_t pa = tile * 16u + ((s.ctrl & 0x10u) << 8) + ((v >> 12) & 7u);
        L->f[j + 2u] = pattern(lo, hi, pa) | (sel << 16);
    }
    // The background palette as 16 bytes in four words, entry 4a + v: palette a's colour v, and for v = 0 the
    // backdrop with bit 6 set (the transparency mark the sprite priority test reads). Wave-uniform.
    // (The tables are written by every active lane, the same 16 bytes: callers may be in lane-divergent code.)
    __device__ void bg_table(uint32_t t[4]) {
        if (bg_stale) {
            const uint4 p = reinterpret_cast<const uint4*>(L->pal)[0];
            const uint32_t b = back();
            L->tab[0] = make_uint4((uni(p.x) & 0x3F3F3F00u) | b, (uni(p.y) & 0x3F3F3F00u) | b,
                                   (uni(p.z) & 0x3F3F3F00u) | b, (uni(p.w) & 0x3F3F3F00u) | b);
            bg_stale = false;
        }
        const uint4 q = L->tab[0];
        t[0] = uni(q.x);
        t[1] = uni(q.y);
        t[2] = uni(q.z);
        t[3] = uni(q.w);
    }
    // 4 background pixels, leftmost in the low byte: kk0..kk0 + 3 of the 8 a slot shifts out from fetches p2 (older),
    // p1 with fine x fx; pixel q is bit 15 - fx - kk0 - q of the two 16-bit plane pairs, with p2's attribute while
    // fx + kk0 + q < 8, else p1's. All four at once: the planes' 4 bits bit-reversed into place and spread one to a
    // byte, the attribute chosen per byte by a mask, and the colours looked up 4 at a time by byte permutes of the
    // palette table.
    __device__ uint32_t shift4(uint32_t p2, uint32_t p1, uint32_t kk0, uint32_t fx, const uint32_t t[4]) {
        const uint32_t sh = fx + kk0;   // 0..11
        const uint32_t lo16 = ((p2 & 0xFFu) << 8) | (p1 & 0xFFu), hi16 = (p2 & 0xFF00u) | ((p1 >> 8) & 0xFFu);
        const uint32_t lo4 = __builtin_bitreverse32(lo16 << (16u + sh)) & 0xFu;   // pixel q at bit q
        const uint32_t hi4 = __builtin_bitreverse32(hi16 << (16u + sh)) & 0xFu;
        const uint32_t val = ((lo4 * 0x00204081u) & 0x01010101u) | (((hi4 * 0x00204081u) & 0x01010101u) << 1);
        const int32_t b = 8 - (int32_t)sh;   // pixels q < b take p2's attribute
        const uint32_t m = b >= 4 ? 0xFFFFFFFFu : b <= 0 ? 0u : (1u << (8 * b)) - 1u;
        // (byte selects by v_perm_b32, whose selector byte k picks byte k of {src0:src1}, src1 the low four: full
        // rate, where spreading a byte by a 32-bit multiply is a quarter-rate instruction)
        const uint32_t attr = __builtin_amdgcn_perm((p1 >> 16) & 3u, (p2 >> 16) & 3u, ~m & 0x04040404u);
        const uint32_t idx = (attr << 2) | val;   // palette entry per byte, 0..15
        const uint32_t sel = idx & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], sel), hi = __builtin_amdgcn_perm(t[3], t[2], sel);
        return __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((idx >> 1) & 0x04040404u));   // entries 8..15 from hi
    }
    __device__ void on_run(const Rs& s, int32_t first, int32_t last, int32_t out, bool pixels) {
        __syncthreads();   // the walker's page and palette writes
        if (lane >= first && lane < last) {
            const uint32_t pk = mmc2 ? L->pages[lane] : 0u;
            fetch_slot(s, v_steps(s.v, (uint32_t)(lane - first)), (uint32_t)lane, mmc2 ? pk : s.chr_lo,
                       mmc2 ? pk : s.chr_hi);
        }
        __syncthreads();
        if (pixels) {
            // lane j writes pixels 4j..4j+3 where they fall in the run's output, [out, out + 8 (last - from))
            const int32_t from = first > 2 ? first : 2, x = 4 * lane;
            if (last > from && x >= out && x < out + 8 * (last - from)) {
                const int32_t k = from + (x - out) / 8;   // the slot that shifts out pixel x
                const int32_t j = k - first;
                const uint32_t p1 = L->f[j >= 1 ? (uint32_t)k + 1u : hb];
                const uint32_t p2 = L->f[j >= 2 ? (uint32_t)k : (j == 1 ? hb : ha)];
                uint32_t t[4];
                bg_table(t);
                L->px[lane] = shift4(p2, p1, (uint32_t)((x - out) & 7), s.fx, t);
            }
            const bool clip = first <= 2 && last > 2 && !(s.mask & 0x02u), bg_off = !(s.mask & 0x08u);
            if (clip || bg_off) {
                __syncthreads();
                if (clip) fill(0, 8);
                if (bg_off) {
                    int32_t f = first - 2, n = last - first;
                    if (f < 0) {
                        n += f;
                        f = 0;
                    }
                    fill(8 * f, 8 * n);
                }
            }
        }
        if (last - first >= 2) {
            ha = (uint32_t)last;
            hb = (uint32_t)last + 1u;
        } else {
            ha = hb;
            hb = (uint32_t)first + 2u;
        }
        __syncthreads();
    }
    __device__ int32_t find_hit(int32_t x, uint32_t bits, int32_t end) {
        const int32_t xi = x + lane;
        const bool hit = lane < 8 && xi < end && ((bits >> (7 - lane)) & 1u) &&
                         !(reinterpret_cast<const uint8_t*>(L->px)[xi] & 0x40u);
        const uint64_t b = __ballot(hit);
        return b ? x + (int32_t)__builtin_ctzll(b) : -1;
    }
    // The lanes' part of FetchSpriteData: lane i is OAM entry i; the first eight on line l + 1 are fetched into the
    // buffer not latched. Returns the ballot of the entries on the line (read the fetch after a sync).
    __device__ uint64_t sprite_fetch_lanes(const Rs& s, int32_t l) {
        const uint32_t ctrl = s.ctrl, h = (ctrl & 0x20u) ? 16u : 8u;
        const uint32_t e = reinterpret_cast<const uint32_t*>(otab)[lane];
        const uint32_t row = (uint32_t)(l - (int32_t)(e & 0xFFu));
        const uint64_t sel = __ballot(row < h);
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(sel >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)sel, 0u));
        const uint32_t target = fetched == drawn ? drawn ^ 1u : fetched;
        if (row < h && rank < 8u) {
            const uint32_t tile = (e >> 8) & 0xFFu;
            const uint32_t table8 = (ctrl & 0x08u) && !(ctrl & 0x20u) ? 0x1000u : 0u;
            const uint32_t base = h == 16u ? ((tile & 1u) << 12) + ((tile & 0xFEu) << 4) : (tile << 4) + table8;
            // the row's offset, row + (row & 8), or with vertical flip (attribute bit 7) 7 (+ 16 for 8x16) minus it:
            // flip = all ones negates it (x ^ flip) - flip and adds the 7 (+ 16)
            const uint32_t r2 = row + (row & 8u), flip = (uint32_t)((int32_t)(e << 8) >> 31);
            const uint32_t pa = (base + (flip & (7u + ((ctrl & 0x20u) >> 1))) + ((r2 ^ flip) - flip)) & 0x1FFFu;
            const uint32_t pk = mmc2 ? L->pages[34 + rank] : 0u;
            const uint32_t lo = mmc2 ? pk : s.chr_lo, hi = mmc2 ? pk : s.chr_hi;
            L->spr[target][rank] = pattern(lo, hi, pa) | (e & 0xFFFF0000u);
        }
        fetched = target;
        return sel;
    }
    // What RefreshSprites needs of the fetch (after the sync).
    __device__ void sprite_fetch_done(Rs& s, uint64_t sel) {
        const uint32_t n = (uint32_t)__builtin_popcountll(sel);
        s.f_n = n < 8u ? n : 8u;
        s.f_blurp = (uint32_t)(sel & 1u);
        if (s.f_n) {
            const uint32_t e0 = uni(L->spr[fetched][0]);
            s.f_bits = (e0 & 0xFFu) | ((e0 >> 8) & 0xFFu);
            s.f_attr = (e0 >> 16) & 0xFFu;
            s.f_x = e0 >> 24;
        }
    }
    __device__ void fetch_sprites(Rs& s, int32_t l) {
        if (mmc2) __syncthreads();   // the walker's page writes
        const uint64_t sel = sprite_fetch_lanes(s, l);
        __syncthreads();
        sprite_fetch_done(s, sel);
    }
    __device__ void latch_table() {
        const uint4 p = reinterpret_cast<const uint4*>(L->pal)[1];
        L->tab[1] = make_uint4(uni(p.x) & 0x3F3F3F3Fu, uni(p.y) & 0x3F3F3F3Fu, uni(p.z) & 0x3F3F3F3Fu,
                               uni(p.w) & 0x3F3F3F3Fu);
        sp_stale = false;
    }
    // RefreshSprites: the fetched line is the one drawn next, with the sprite palette of the moment (read by the next
    // line's compose, after its syncs).
    __device__ void latch_sprites(const Rs& s) {
        drawn = fetched;
        drawn_n = s.f_n;
        if (sp_stale) latch_table();
    }
    // CopySprites (with sprites on at the line's end and a latched line waiting) over the background pixels w of
    // this lane, greyscale while rendering, and the observation row (rl/csrc/nes_machine.cuh:133-155: lines 8..231,
    // x 8..247) with the line's emphasis (patch:1637-1661). Clears the lane's part of the sprite line.
    __device__ void sprite_table(uint32_t t[4]) {
        const uint4 q = L->tab[1];
        t[0] = uni(q.x);
        t[1] = uni(q.y);
        t[2] = uni(q.z);
        t[3] = uni(q.w);
    }
    // spt: the latched sprite palette (sprite_table). The line's emphasis is the caller's (the mask at this point).
    __device__ void compose(Rs& s, int32_t l, uint32_t w, uint8_t* obs, const uint32_t spt[4]) {
        const bool expanded = s.spork != 0, sprites = (s.mask & 0x10u) && expanded;
        if (sprites) s.spork = 0;
        const uint32_t keep = (s.mask & 0x01u) && rs_rendering(s) ? 0x30u : 0x3Fu;
        if (expanded) {
            const uint4 sp = reinterpret_cast<const uint4*>(L->sp)[lane];
            reinterpret_cast<uint4*>(L->sp)[lane] = make_uint4(0u, 0u, 0u, 0u);
            if (sprites) {
                // the four pixels at once, one per byte: a sprite pixel (value != 0) shows in front, or behind a
                // transparent background pixel (bit 6, the backdrop mark), except in the left 8 with sprite
                // clipping; its colour from the latched sprite palette by byte permutes (entry = palette << 2 | value)
                const uint32_t eb = (sp.x & 0xFFu) | ((sp.y & 0xFFu) << 8) | ((sp.z & 0xFFu) << 16) | (sp.w << 24);
                const uint32_t opaque = (eb | (eb >> 1)) & 0x01010101u;
                const uint32_t front = ~(eb >> 7) & 0x01010101u, clear_bg = (w >> 6) & 0x01010101u;
                const bool clipped = !(s.mask & 0x04u) && lane < 2;
                const uint32_t show = clipped ? 0u : opaque & (front | clear_bg);
                const uint32_t sel = eb & 0x07070707u;
                const uint32_t lo = __builtin_amdgcn_perm(spt[1], spt[0], sel), hi = __builtin_amdgcn_perm(spt[3], spt[2], sel);
                const uint32_t col = __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((eb >> 1) & 0x04040404u));
                w = __builtin_amdgcn_perm(col, w, 0x03020100u | (show << 2));   // the shown bytes from col
            }
        }
        if (l < 8) return;
        w &= keep * 0x01010101u;
        const int32_t y = l - 8;
        if (lane >= 2 && lane < 62) reinterpret_cast<uint32_t*>(obs + y * RLE_OBS_W)[lane - 2] = w;
    }
    // Emphasis of rows y0 .. y1 - 1 (the lines' mask bits 5-7).
    __device__ void emphasis(uint8_t* emph, int32_t y0, int32_t y1, uint32_t mask) {
        for (int32_t y = y0 + lane; y < y1; y += 64) emph[y] = (uint8_t)((mask >> 5) & 7u);
    }
    // The line's sprite-0 check (replay_dev.h rs_check at the line's end, where the whole line is drawn): the first
    // pixel in [sphitx, min(sphitx + 8, 255)) where sprite 0's pixel is set and the background pixel is not
    // transparent (bit 6, the backdrop mark), over the background pixels w the lanes hold (4 each).
    __device__ void check_hit(Rs& s, uint32_t w) {
        const int32_t x0 = s.sphitx, end = x0 + 8 < 255 ? x0 + 8 : 255;
        uint32_t first = 4u;
        for (uint32_t q = 0; q < 4u; ++q) {
            const int32_t x = 4 * lane + (int32_t)q;
            const bool in = x >= x0 && x < end;
            const uint32_t bit = in ? (s.sphit_bits >> (uint32_t)(7 - (x - x0))) & 1u : 0u;
            if (first == 4u && bit && !((w >> (8u * q)) & 0x40u)) first = q;
        }
        const uint64_t b = __ballot(first < 4u);
        if (b) {
            const int ln = (int)__builtin_ctzll(b);
            s.hit = 1;
            s.hit_x = 4 * ln + __builtin_amdgcn_readlane((int)first, ln);
            s.sphitx = kNoCheck;
        }
    }
    // Lines l .. stop - 1, a run with no write from the first one's lead-in to the last one's end (and no MMC2
    // latches): each line is one run of the 34 slots with the state as it is, the sprite-0 check (if one is due)
    // against the drawn line, FetchSpriteData, Fixit1/Fixit2 and RefreshSprites in closed form. ctrl, mask, the
    // palette, the CHR pages and the nametable map hold for the whole run, so what follows from them is set up once:
    //   - background: lane j fetches tile slot (j + 1) / 2, so lanes 2i and 2i + 1 hold slots i and i + 1 between
    //     them, the two fetches that lane 2i's pixels 8i..8i+3 and lane 2i + 1's 8i+4..8i+7 shift out (pixel x from
    //     slots x / 8 and x / 8 + 1), and one swap within the lane pair (DPP) gives each lane both. The tile and
    //     attribute (with CHR ROM the row of tiles' pair index) are read again only when v's row of tiles changes
    //     (every 8 lines), the pattern row every line;
    //   - sprites: lane i keeps OAM entry i and its pattern row base (with CHR ROM its row 0's pair index);
    //     FetchSpriteData is one ballot over the lanes;
    //   - the lanes expand this line's sprites, sync once, and each composes its 4 pixels in registers;
    //   - the run's state (v, the latched sprite line, the sprite-0 check) stays in scalar registers, with selects
    //     and masks rather than lane-divergent branches: the CU's scalar unit is what the emulator's waves need.
    // With rendering off the lines are the backdrop: nothing is fetched, v stays, no sprite is drawn and no sprite-0
    // check can hit (the backdrop is transparent).
    // kSpr: sprites on (mask bit 4) for the run.
    template <bool kPairs, bool kSpr>
    __device__ void fast_run(Rs& s, int32_t l, int32_t stop, uint8_t* obs, uint8_t* emph) {
        uint32_t t[4];
        bg_table(t);
        const uint32_t back4 = (t[0] & 0xFFu) * 0x01010101u;
        const uint32_t mask = s.mask;
        if (!rs_rendering(s)) {
            const uint32_t row4 = back4 & 0x3F3F3F3Fu;
            for (int32_t y = (l > 8 ? l : 8) - 8; y < stop - 8; ++y)
                if (lane >= 2 && lane < 62) reinterpret_cast<uint32_t*>(obs + y * RLE_OBS_W)[lane - 2] = row4;
            emphasis(emph, (l > 8 ? l : 8) - 8, stop - 8, mask);
            s.sphitx = kNoCheck;
            return;
        }
        const uint32_t ctrl = s.ctrl, h = (ctrl & 0x20u) ? 16u : 8u, ptab = (ctrl & 0x10u) << 8;
        const bool bg_on = (mask & 0x08u) && (lane >= 2 || (mask & 0x02u)), spr_on = kSpr;
        // this lane's OAM entry: its pattern row is sb + row (+ 8 for the lower tile of 8x16), vertical flip negating
        // the row (flip = all ones: (r ^ flip) - flip, and sb adds the 7 or 23)
        const uint32_t e = reinterpret_cast<const uint32_t*>(otab)[lane];
        const uint32_t st = (e >> 8) & 0xFFu, table8 = (ctrl & 0x08u) && !(ctrl & 0x20u) ? 0x1000u : 0u;
        const uint32_t flip = (uint32_t)((int32_t)(e << 8) >> 31);
        const uint32_t sb = (h == 16u ? ((st & 1u) << 12) + ((st & 0xFEu) << 4) : (st << 4) + table8) +
                            (flip & (7u + ((ctrl & 0x20u) >> 1)));
        const uint32_t slot = ((uint32_t)lane + 1u) >> 1, kk0 = ((uint32_t)lane & 1u) * 4u;
        // (kPairs) the entry's rows in one 1 KB page: row r's pair at sp_i0 + r, or flipped sp_i0 + h - 1 - r. With
        // pb its row 0's pattern address (16-aligned, 32 for 8x16), the pattern of row r is at pb + r for 8x8, pb + r
        // + (r & 8) for 8x16 (the tile after), whose pair index is that of pb plus r; flipped the rows run backwards.
        const uint32_t sp_i0 = kPairs ? pairs_index(s.chr_lo, s.chr_hi, sb - (flip & (7u + ((ctrl & 0x20u) >> 1)))) +
                                            (flip & (h - 1u))
                                      : 0u;
        // the latched sprite palette. With sprites on, the line before the run ended with RefreshSprites: it latched
        // the palette as it is now, or latched nothing (no sprite is drawn before a latch in the run, which takes this
        // same palette), so the table can be brought up to date here. With sprites off nothing is latched or drawn in
        // the run, and the table keeps the palette of the last latch for the lines after it.
        if (spr_on && sp_stale) latch_table();
        uint32_t spt[4];
        sprite_table(spt);
        // what else the run holds fixed: greyscale (rendering is on), the left-8 sprite clip, t's horizontal bits
        const uint32_t keep4 = (mask & 0x01u) ? 0x30303030u : 0x3F3F3F3Fu;
        const uint32_t show_m = !(mask & 0x04u) && lane < 2 ? 0u : 0xFFFFFFFFu;
        const uint32_t t_h = s.t & 0x041Fu, kk = (uint32_t)lane >> 3, px = (uint32_t)lane & 7u;
        // the row's 60 words are stored by all 64 lanes: lanes 0 and 1 store lane 2's word, 62 and 63 lane 61's
        const int32_t ox = 4 * (lane < 2 ? 0 : lane > 61 ? 59 : lane - 2);
        // The run's state in registers, written back after it. The two sprite buffers are 0 and 1, so the one a
        // fetch fills (the one not latched) is drawn ^ 1. spork: a line was latched at the end of the line before
        // (with sprites on the only way it is set in the run; with sprites off nothing is drawn, so the latched line
        // is not expanded: the sprite line stays clear, as the compose would leave it).
        uint32_t vl = s.v, dr = drawn, dr_n = drawn_n, spork = s.spork, tgt = drawn ^ 1u;
        uint32_t hit = s.hit, sp_bits = s.sphit_bits, f_bits = s.f_bits, f_attr = s.f_attr, f_x = s.f_x;
        int32_t sphitx = s.sphitx, hit_x = s.hit_x;
        uint64_t sel = 0;
        uint32_t key = 0xFFFFFFFFu, tb = 0, tsel = 0, vline = vl;
        const int32_t l0 = l;
        for (; l < stop; ++l) {
            vline = vl;
            if ((vl & 0x0FFFu) != key) {   // a new row of tiles (or the run's first line)
                key = vl & 0x0FFFu;
                const uint32_t vs = v_steps(vl, slot);
                const uint32_t ntb = 0x2000u | (vs & 0x0C00u), col = vs & 31u;
                const uint32_t tile = ntab[nt_slot(s.nt_map, ntb | (vs & 0x3FFu))];
                const uint32_t at = ntab[nt_slot(s.nt_map, ntb | 0x3C0u | (col >> 2) | ((vs & 0x380u) >> 4))];
                tsel = ((at >> ((col & 2u) | ((vs & 0x40u) >> 4))) & 3u) << 16;
                tb = tile * 16u + ptab;
                if constexpr (kPairs) tb = pairs_index(s.chr_lo, s.chr_hi, tb);   // (fine y adds to the index)
            }
            // FetchSpriteData for line l + 1 into buffer tgt (every lane fetches its entry's row, only the first eight
            // on the line keep it)
            const uint32_t row = (uint32_t)(l - (int32_t)(e & 0xFFu));
            sel = __ballot(row < h);
            const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(sel >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)sel, 0u));
            uint32_t spp;
            if constexpr (kPairs) {
                const uint32_t rc = row < h ? row : 0u;   // (an entry off the line reads its row 0: in bounds)
                spp = chr_pairs[sp_i0 + ((rc ^ flip) - flip)];
            } else {
                const uint32_t r2 = row + (row & 8u);
                spp = pattern_of<kPairs>(s.chr_lo, s.chr_hi, (sb + ((r2 ^ flip) - flip)) & 0x1FFFu);
            }
            const uint32_t sp = spp | (e & 0xFFFF0000u);
            const uint32_t mine = (kPairs ? (uint32_t)chr_pairs[tb + ((vl >> 12) & 7u)]
                                          : pattern_of<kPairs>(s.chr_lo, s.chr_hi, tb + ((vl >> 12) & 7u))) | tsel;
            const uint32_t other = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0xB1, 0xF, 0xF, false);   // lane ^ 1
            // (the lanes that keep nothing store into their own word of the line buffer, unused by this path)
            const uint32_t slot_k = rank + (row < h ? 0u : 8u);
            *(slot_k < 8u ? &L->spr[tgt][slot_k] : &L->px[lane]) = sp;
            const uint32_t fetched_now = tgt;
            const uint32_t bgw = shift4(lane & 1 ? other : mine, lane & 1 ? mine : other, kk0, s.fx, t);
            uint32_t w = bg_on ? bgw : back4;
            if (sphitx != kNoCheck) {   // (check_hit on the run's registers: the background pixels)
                const int32_t end = sphitx + 8 < 255 ? sphitx + 8 : 255;
                uint32_t first = 4u;
                for (uint32_t q = 0; q < 4u; ++q) {
                    const int32_t x = 4 * lane + (int32_t)q;
                    const bool in = x >= sphitx && x < end;
                    const uint32_t bit = in ? (sp_bits >> (uint32_t)(7 - (x - sphitx))) & 1u : 0u;
                    if (first == 4u && bit && !((w >> (8u * q)) & 0x40u)) first = q;
                }
                const uint64_t hb_ = __ballot(first < 4u);
                if (hb_) {
                    const int ln = (int)__builtin_ctzll(hb_);
                    hit = 1;
                    hit_x = 4 * ln + __builtin_amdgcn_readlane((int)first, ln);
                }
            }
            if (spr_on && spork) {
                // this line's sprites: lane 8k + p expands pixel p of latched sprite k (expand_sprites), every lane
                // issuing its LDS max, a zero (no change) where there is nothing to draw
                const uint32_t es = L->spr[dr][kk];
                const uint32_t attr = (es >> 16) & 0xFFu, b = (attr & 0x40u) ? px : 7u - px;
                const uint32_t x = (es >> 24) + px;
                uint32_t val = ((es >> b) & 1u) | (((es >> (8u + b)) & 1u) << 1);
                // (k < drawn_n and x < 256 as sign masks)
                val &= (uint32_t)((int32_t)(x - 256u) >> 31) & (uint32_t)((int32_t)(kk - dr_n) >> 31);
                const uint32_t ent = ((7u - kk) << 8) | ((attr & 0x20u) << 2) | ((attr & 3u) << 2) | val;
                atomicMax(&L->sp[x & 0xFFu], ent & (0u - (val < 1u ? val : 1u)));
                __syncthreads();
                // compose: the sprite pixels over the background, the lane's part of L->sp cleared
                const uint4 spq = reinterpret_cast<const uint4*>(L->sp)[lane];
                reinterpret_cast<uint4*>(L->sp)[lane] = make_uint4(0u, 0u, 0u, 0u);
                const uint32_t eb = (spq.x & 0xFFu) | ((spq.y & 0xFFu) << 8) | ((spq.z & 0xFFu) << 16) | (spq.w << 24);
                const uint32_t opaque = (eb | (eb >> 1)) & 0x01010101u;
                const uint32_t front = ~(eb >> 7) & 0x01010101u, clear_bg = (w >> 6) & 0x01010101u;
                const uint32_t show = opaque & (front | clear_bg) & show_m;
                const uint32_t ssel = eb & 0x07070707u;
                const uint32_t lo = __builtin_amdgcn_perm(spt[1], spt[0], ssel), hi = __builtin_amdgcn_perm(spt[3], spt[2], ssel);
                const uint32_t col = __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((eb >> 1) & 0x04040404u));
                w = __builtin_amdgcn_perm(col, w, 0x03020100u | (show << 2));
            }
            if (l >= 8) {
                uint32_t wo = w & keep4;
                wo = (uint32_t)__builtin_amdgcn_update_dpp((int)wo, (int)wo, 0xEA, 0x1, 0x1, false);   // 0-3: [2,2,2,3]
                wo = (uint32_t)__builtin_amdgcn_update_dpp((int)wo, (int)wo, 0x54, 0x8, 0x8, false);   // 60-63: [0,1,1,1]
                *reinterpret_cast<uint32_t*>(obs + (l - 8) * RLE_OBS_W + ox) = wo;
            }
            // the end of the line: Fixit1 and Fixit2 (v from t horizontally), RefreshSprites
            sphitx = kNoCheck;
            if (__builtin_expect((vl & 0x7000u) == 0x7000u, 0)) vl = y_step(vl);
            else vl += 0x1000u;
            vl = (vl & 0x7BE0u) | t_h;
            if (spr_on) {
                const uint32_t n = (uint32_t)__builtin_popcountll(sel);
                spork = n < 1u ? n : 1u;
                dr_n = spork ? (n < 8u ? n : 8u) : dr_n;
                dr = spork ? fetched_now : dr;
            }
            if (__builtin_expect((uint32_t)sel & 1u, 0)) {   // sprite 0 fetched for the next line: what RefreshSprites keeps
                const uint32_t e0 = (uint32_t)__builtin_amdgcn_readlane((int)sp, 0);
                f_bits = (e0 & 0xFFu) | ((e0 >> 8) & 0xFFu);
                f_attr = (e0 >> 16) & 0xFFu;
                f_x = e0 >> 24;
                if (spr_on && !hit && f_bits) {
                    sphitx = (int32_t)f_x;
                    sp_bits = (f_attr & 0x40u) ? __builtin_bitreverse32(f_bits) >> 24 : f_bits;
                }
            }
            tgt = dr ^ 1u;
            fetched = fetched_now;
        }
        emphasis(emph, (l0 > 8 ? l0 : 8) - 8, stop - 8, mask);
        // the state after the run (sprite_fetch_done, latch_sprites and the check's on the last line)
        const uint32_t n_last = (uint32_t)__builtin_popcountll(sel);
        s.v = vl;
        s.f_n = n_last < 8u ? n_last : 8u;
        s.f_blurp = (uint32_t)(sel & 1u);
        s.f_bits = f_bits;
        s.f_attr = f_attr;
        s.f_x = f_x;
        s.spork = spork;
        s.hit = hit;
        s.hit_x = hit_x;
        s.sphitx = sphitx;
        s.sphit_bits = sp_bits;
        drawn = dr;
        drawn_n = dr_n;
        // the last line's slots 32 and 33, where a line with writes after the run starts from (F[34], F[35]): v
        // before the line's Fixit1/Fixit2
        if (lane < 2) fetch_slot(s, v_steps(vline, 32u + (uint32_t)lane), 32u + (uint32_t)lane, s.chr_lo, s.chr_hi);
        ha = 34u;
        hb = 35u;
    }
};

// One console-frame's picture into obs (224 rows of 240 colour indices, lines 8..231, x 8..247) and emph (the rows'
// emphasis bits), replayed from its frame log (header and events) over its nametables and OAM as of the frame's
// vblank stop (nt, oam: LDS) and the cartridge's CHR (chr_ram on carts with CHR RAM), by the 64 lanes of one wave with
// the scratch L.
template <bool kScalarLog>
__device__ __forceinline__ void draw_frame(RenderScratch* L, uint8_t* nt, uint8_t* oam, const uint32_t* log,
                                           uint32_t log_n, const Cart& cart, const uint8_t* chr_ram, uint8_t* obs,
                                           uint8_t* emph, int lane) {
    if (lane < 8) reinterpret_cast<uint32_t*>(L->pal)[lane] = log[6 + lane];
    if (lane < 2) L->f[lane] = 0;
    if (lane < 16) L->spr[lane >> 3][lane & 7] = 0;
    reinterpret_cast<uint4*>(L->sp)[lane] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    const bool mmc2 = cart.board == NES_BOARD_MMC2;
    RenderSink<kScalarLog> sink{L, nt, oam, log, cart.chr, chr_ram, cart.chr_pairs, lane, mmc2, 0u, 1u, 0u, 0u, 0u,
                                true, true};
    Rs s;
    rs_load(s, sink, log, uni(log_n), mmc2 ? cart.chr_pages1 : 0u);
    rs_begin_frame(s, sink);
    for (int32_t l = 0; l < 232; ++l) {
        if (!mmc2 && s.next >= (l + 1) * 341 - NES_LINE_LEAD) {
            // lines l .. stop - 1 end before the next write's line (its lead-in included)
            const int32_t stop = s.next >= 232 * 341 - NES_LINE_LEAD ? 232 : (s.next + NES_LINE_LEAD) / 341;
            const bool spr = (s.mask & 0x10u) != 0;
            if (sink.chr_pairs) {
                if (spr) sink.template fast_run<true, true>(s, l, stop, obs, emph);
                else sink.template fast_run<true, false>(s, l, stop, obs, emph);
            } else {
                if (spr) sink.template fast_run<false, true>(s, l, stop, obs, emph);
                else sink.template fast_run<false, false>(s, l, stop, obs, emph);
            }
            l = stop - 1;
            continue;
        }
        rs_line(s, sink, l, true);
        uint32_t spt[4];
        sink.sprite_table(spt);
        sink.compose(s, l, L->px[lane], obs, spt);
        if (l >= 8) sink.emphasis(emph, l - 8, l - 7, s.mask);
        rs_end_of_line(s, sink, l, true);
    }
}

}  // namespace nd
