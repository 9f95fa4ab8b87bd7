// Host-side translation of a fixed-PRG cartridge's 6502 code (NROM, CNROM) into blocks of straight-line calls of the
// interpreter's per-opcode handlers (wave_dev.h fx<B, D>) with the operand and the pc as constants, so that the
// compiler folds the operand addressing and the cycle count, and a block runs without the fetch-table load, the
// opcode dispatch or the burst counter test between its instructions. The blocks are compiled into a copy of the
// console-frame kernel at run time (hiprtc, rlenv_hip.hip), once per cartridge.
//
// Blocks start at leaders: the reset, NMI and IRQ vectors, the targets of branches, JMP and JSR, the instruction
// after a branch or a JSR (the fall-through and the return point), and the instruction after one that always needs
// the generic step. Code is found by following those from the vectors (a recursive descent over CPU addresses
// $8000-$FFFD); the byte sequence each leader starts is decoded on its own, so overlapping instruction streams are
// fine. A block ends at a branch, a jump, a call or a return, before an instruction that always needs the generic
// step (I/O other than $2002 reads, $4016 and PRG RAM, a jump to itself, an unofficial opcode), at the next leader, or after
// kJitMaxBlock instructions; blocks are made in address order until kJitMaxInstructions. A copy of the fetch table
// marks each block's first entry with the key kBlockKey + block index; at any other address the interpreter runs as
// before.
//
// Exactness: a block runs only when the burst counter has room for the most cycles its instructions can take (so no
// instruction inside it ends the burst early); otherwise its first instruction runs alone with the interpreter's
// own test. An instruction that needs the generic step at run time (an indexed access that lands on I/O) leaves the
// block before any state change, as in the interpreter. Each handler is the interpreter's own, so a block changes
// the console exactly as the same instructions interpreted one by one.
#pragma once
#include <stdint.h>

#include <cstdio>
#include <set>
#include <string>
#include <vector>

#include "optab.h"

namespace nd {

constexpr uint32_t kJitMaxBlock = 48;            // instructions per block at most
constexpr uint32_t kJitMaxInstructions = 8192;   // instructions in all blocks of a cartridge at most

struct JitProgram {
    std::string cases;                    // the blocks as the cases of the burst loop's switch (wave_dev.h)
    std::vector<uint32_t> leader_addr;    // block i starts at CPU address leader_addr[i]
    uint32_t instructions = 0;            // instructions in all blocks
};

// Whether the instruction (op, b1, b2) at CPU address a always needs the generic step (fx returns kGeneric whatever
// the registers): its memory class is fixed by a constant address.
// board: the image's board, whose bank writes the fast path may take (wave_dev.h map_write_ok, decided at run time: the
// block leaves before one it does not take): MMC3 at $8000-$9FFF, MMC2 at $A000-$AFFF, MMC1 and UxROM anywhere at
// $8000+.
inline bool jit_fast_bank_write(uint32_t board, uint32_t ea) {
    if (ea < 0x8000u) return false;
    if (board == NES_BOARD_MMC3) return (ea & 0xE000u) == 0x8000u;
    if (board == NES_BOARD_MMC2) return (ea & 0xF000u) == 0xA000u;
    return board == NES_BOARD_MMC1 || board == NES_BOARD_UXROM;
}
inline bool jit_always_generic(uint32_t a, uint32_t op, uint32_t b1, uint32_t b2, uint32_t board = NES_BOARD_NROM) {
    const uint32_t d = kOptab.t[op], mode = d & 15u, grp = (d >> 8) & 15u;
    const bool rd = (d & D_READ) != 0, wr = (d & D_WRITE) != 0;
    if (grp == G_ILL || grp == G_BRK) return true;
    const uint32_t ea = b1 | (b2 << 8);
    if (grp == G_JMP) {
        if (mode == M_ABS) return ea == a;   // the idle loop
        const uint32_t a1 = (ea & 0xFF00u) | ((ea + 1u) & 0xFFu);
        return (ea >= 0x2000u && ea < 0x8000u) || (a1 >= 0x2000u && a1 < 0x8000u);
    }
    if (mode != M_ABS || grp == G_JSR) return false;
    const bool prg_ram = ea >= 0x6000u && ea < 0x8000u;   // served by the fast path except on MMC1 (decided then)
    // a PPU register write: the fast path takes those of a burst between vblank and the pre-render line (wave_dev.h
    // ppu_write_quiet); the others end the burst at run time
    const bool ppu = ea >= 0x2000u && ea < 0x4000u;
    if (rd && wr) return ea >= 0x2000u && !prg_ram;
    if (wr) return ea >= 0x2000u && ea != 0x4016u && !ppu && !prg_ram && !jit_fast_bank_write(board, ea);
    if (rd) return !(ea < 0x2000u || ea >= 0x8000u || ea == 0x4016u || (ea & 0xE007u) == 0x2002u || prg_ram);
    return false;
}

// An absolute store to a PPU register: the last instruction of its block, so that when it needs the generic step
// (outside a quiet burst: wave_dev.h ppu_write_quiet) the burst resumes at a block's start, the instruction after it.
inline bool jit_ppu_store(uint32_t op, uint32_t b1, uint32_t b2) {
    const uint32_t d = kOptab.t[op], ea = b1 | (b2 << 8);
    return (d & 15u) == M_ABS && (d & D_WRITE) && !(d & D_READ) && ((d >> 8) & 15u) != G_JMP &&
           ((d >> 8) & 15u) != G_JSR && ea >= 0x2000u && ea < 0x4000u;
}

// The most a fast instruction of opcode op takes off the burst counter (wave_dev.h jit_maxtake).
inline uint32_t jit_take_max(uint32_t op) {
    const uint32_t d = kOptab.t[op];
    return ((((d >> 4) & 15u) + ((d & D_PEN) ? 1u : 0u) + (((d >> 8) & 15u) == G_BR ? 2u : 0u)) << 14) - 1u;
}

// A status poll: a block of two instructions, a read of $2002 (BIT, LDA, LDX or LDY absolute, at any mirror) and a
// branch back to the read that the read's own side effect cannot turn: BPL (taken while bit 7, the vblank flag, is
// clear, and the read leaves it clear), BVC or BVS (bit 6, the sprite-0 flag, which a read does not touch). The
// status changes only at PPU events, which a burst stops short of, and a read after the first leaves the console as
// it found it (the vblank flag and the write toggle already clear, the open bus the same), so within a burst the
// iterations after the first are alike: the translation takes as many of them at once as the burst's room allows.
// The counter then stands where iterating would leave it (below the block's room), and the block goes on as before.
// BMI is not one: taken, its read saw the vblank flag set and cleared it, so the next iteration falls through.
inline std::string jit_poll_skip(uint32_t op0, uint32_t addr, uint32_t op1, bool to_self, uint32_t cyc_taken) {
    const bool poll = to_self && (op0 == 0x2Cu || op0 == 0xADu || op0 == 0xAEu || op0 == 0xACu) &&
                      (addr & 0xE007u) == 0x2002u && (op1 == 0x10u || op1 == 0x50u || op1 == 0x70u);
    if (!poll) return std::string();
    const uint32_t room = jit_take_max(op0) + jit_take_max(op1);
    const uint32_t iter = ((((kOptab.t[op0] >> 4) & 15u) + cyc_taken) << 14) - 2u;   // two instructions
    char buf[160];
    snprintf(buf, sizeof buf, "if (v >= 0x%Xu) v -= ((v - 0x%Xu) / 0x%Xu + 1u) * 0x%Xu; ", room, room, iter, iter);
    return buf;
}

// The blocks of a fixed PRG image: the CPU sees byte prg[a & (size - 1)] at $8000-$FFFF (size 16 or 32 KB).
inline JitProgram jit_translate_fixed(const std::vector<uint8_t>& prg) {
    const uint32_t mask = (uint32_t)prg.size() - 1u;
    auto rd = [&](uint32_t a) { return (uint32_t)prg[a & mask]; };
    auto rd16 = [&](uint32_t a) { return rd(a) | (rd(a + 1u) << 8); };
    auto in_prg = [](uint32_t a) { return a >= 0x8000u && a <= 0xFFFDu; };
    auto generic = [&](uint32_t a) { return jit_always_generic(a, rd(a), rd(a + 1u), rd(a + 2u)); };
    auto grp_of = [&](uint32_t a) { return (kOptab.t[rd(a)] >> 8) & 15u; };
    auto next_of = [&](uint32_t a) { return a + instr_len(kOptab.t[rd(a)] & 15u); };
    auto target_of = [&](uint32_t a) { return next_of(a) + (uint32_t)(int32_t)(int8_t)rd(a + 1u); };

    // 1. leaders: every instruction reachable from the vectors, new leaders on the way
    std::set<uint32_t> leaders, seen;
    std::vector<uint32_t> work;
    auto entry = [&](uint32_t a) {
        if (in_prg(a) && leaders.insert(a).second) work.push_back(a);
    };
    entry(rd16(0xFFFAu));
    entry(rd16(0xFFFCu));
    entry(rd16(0xFFFEu));
    while (!work.empty()) {
        uint32_t a = work.back();
        work.pop_back();
        while (in_prg(a) && seen.insert(a).second) {
            const uint32_t grp = grp_of(a), mode = kOptab.t[rd(a)] & 15u;
            if (generic(a)) {
                if (grp != G_ILL && grp != G_BRK && grp != G_JMP) entry(next_of(a));
                break;
            }
            if (jit_ppu_store(rd(a), rd(a + 1u), rd(a + 2u))) {
                entry(next_of(a));
                break;
            }
            if (grp == G_BR) {
                entry(target_of(a));
                entry(next_of(a));
                break;
            }
            if (grp == G_JMP) {
                if (mode == M_ABS) entry(rd16(a + 1u));
                break;
            }
            if (grp == G_JSR) {
                entry(rd16(a + 1u));
                entry(next_of(a));
                break;
            }
            if (grp == G_RTS || grp == G_RTI) break;
            a = next_of(a);
        }
    }

    // 2. each leader's instructions (none for a leader that starts with an always-generic instruction)
    struct Block { uint32_t start; std::vector<uint32_t> ins; uint32_t stop; };   // stop: the address after it
    std::vector<Block> blocks;
    for (uint32_t start : leaders) {
        Block b{start, {}, start};
        uint32_t a = start;
        for (;;) {
            if (!in_prg(a) || (a != start && leaders.count(a)) || b.ins.size() == kJitMaxBlock || generic(a)) break;
            b.ins.push_back(a);
            const uint32_t grp = grp_of(a);
            a = next_of(a);
            if (grp == G_BR || grp == G_JMP || grp == G_JSR || grp == G_RTS || grp == G_RTI) break;
        }
        b.stop = a;
        if (!b.ins.empty()) blocks.push_back(b);
    }

    // 3. block indices in address order, within the instruction cap
    JitProgram p;
    std::vector<int> id_of(0x10000, -1);
    std::vector<const Block*> kept;
    for (const Block& b : blocks) {
        if (p.instructions + b.ins.size() > kJitMaxInstructions) break;
        id_of[b.start] = (int)kept.size();
        kept.push_back(&b);
        p.leader_addr.push_back(b.start);
        p.instructions += (uint32_t)b.ins.size();
    }

    // 4. the cases. A block's exit jumps straight to the block at a when that cannot close a loop with several entries
    // (every block is also entered from the loop's switch): to itself, or forward to a later address, so that the
    // control flow stays reducible. Any other exit goes back to the loop, which fetches the entry at the new pc.
    auto go = [&](uint32_t from, uint32_t a) {
        return in_prg(a) && id_of[a] >= 0 && a >= from ? "goto JB_" + std::to_string(id_of[a]) + ";"
                                                       : std::string("continue;");
    };
    auto operand = [&](uint32_t x) {   // the fetch table's decoded operand word (rlenv_hip.hip fetch_entry, NROM)
        const uint32_t mode = kOptab.t[rd(x)] & 15u, grp = grp_of(x);
        if (mode == M_IMM || mode == M_ZP || mode == M_ZPX || mode == M_ZPY || mode == M_IZX || mode == M_IZY)
            return rd(x + 1u);
        if (mode == M_REL) return (target_of(x) & 0x1FFFFu) << 3;
        if ((grp == G_JMP && mode == M_ABS) || grp == G_JSR) return rd16(x + 1u) << 3;
        return rd16(x + 1u);
    };
    char buf[200];
    for (size_t i = 0; i < kept.size(); ++i) {
        const Block& b = *kept[i];
        const uint32_t last = b.ins.back(), grp = grp_of(last), mode = kOptab.t[rd(last)] & 15u;
        std::string end;
        bool branch_end = false;
        if (grp == G_BR) {
            // the block's branch itself: taken or not, each with its cycle count and next pc as constants (pc and
            // target times 8, a page crossing when they differ in bits 8-15; fx's own arithmetic)
            const uint32_t tgt = (target_of(last) & 0x1FFFFu) << 3, nxt = (last + 2u) << 3;
            const uint32_t cyc = (kOptab.t[rd(last)] >> 4) & 15u, cross = ((nxt ^ tgt) & (0xFF00u << 3)) ? 1u : 0u;
            snprintf(buf, sizeof buf, "if (br_taken<kOptab.t[0x%02Xu]>(h)) { v -= 0x%Xu; h.pc = 0x%Xu; ", rd(last),
                     ((cyc + 1u + cross) << 14) - 1u, tgt);
            const std::string skip = b.ins.size() == 2u ? jit_poll_skip(rd(b.start), rd16(b.start + 1u), rd(last),
                                                                         target_of(last) == b.start, cyc + 1u + cross)
                                                        : std::string();
            end = buf + skip + go(b.start, target_of(last));
            snprintf(buf, sizeof buf, " } v -= 0x%Xu; h.pc = 0x%Xu; ", (cyc << 14) - 1u, nxt);
            end += buf + go(b.start, b.stop);
            branch_end = true;
        } else if (grp == G_JMP || grp == G_JSR) {
            end = mode == M_ABS ? go(b.start, rd16(last + 1u)) : std::string("continue;");
        } else if (grp == G_RTS || grp == G_RTI) {
            end = "continue;";
        } else {
            end = go(b.start, b.stop);   // the next leader, or back to the loop at an always-generic instruction
        }
        snprintf(buf, sizeof buf, "case 0x%Xu: JB_%zu: {   // $%04X, %zu instructions\n", kBlockKey + (uint32_t)i, i,
                 b.start, b.ins.size());
        p.cases += buf;
        std::string mx;
        for (uint32_t x : b.ins) {
            snprintf(buf, sizeof buf, "%sjit_maxtake(0x%02Xu)", mx.empty() ? "" : " + ", rd(x));
            mx += buf;
        }
        snprintf(buf, sizeof buf, ") { JIT_ONE(0x%02Xu, 0x%Xu, 0x%Xu) }\n", rd(b.start), b.start << 3,
                 operand(b.start));
        p.cases += "    if (v < " + mx + buf;
        for (size_t j = 0; j + (branch_end ? 1u : 0u) < b.ins.size(); ++j) {
            const uint32_t x = b.ins[j];
            snprintf(buf, sizeof buf, "    JIT_STEP(0x%02Xu, 0x%Xu, 0x%Xu)\n", rd(x), x << 3, operand(x));
            p.cases += buf;
        }
        p.cases += "    " + end + "\n}\n";
    }
    return p;
}

// The blocks of a banked PRG image (MMC1, UxROM, MMC3, MMC2), by PRG offset: which bank a window holds is known only
// at run time, so a block is a run of one 8 KB page, pcs its PRG offset x 8 (the fetch table's index on these
// boards, wave_dev.h), and only branches inside the page and falls into the next leader of the page jump straight;
// jumps, calls and returns map their target through the page table at run time and go back to the loop. Leaders:
// the vectors' offsets in the last two pages (the banks fixed at $C000-$FFFF at power-on), then, for every JMP or JSR
// target found, its offset within its 8 KB window in every page (any bank may be mapped there), and inside a page
// the branch targets, return points and the instruction after an always-generic one. Blocks are kept in the order
// they are found from the vectors first, within kJitMaxInstructions.
inline JitProgram jit_translate_banked(const std::vector<uint8_t>& prg, uint32_t board) {
    const uint32_t size = (uint32_t)prg.size(), pages = size >> 13;
    auto rd = [&](uint32_t o) { return o < size ? (uint32_t)prg[o] : 0u; };
    auto rd16 = [&](uint32_t o) { return rd(o) | (rd(o + 1u) << 8); };
    auto len_of = [&](uint32_t o) { return instr_len(kOptab.t[rd(o)] & 15u); };
    auto grp_of = [&](uint32_t o) { return (kOptab.t[rd(o)] >> 8) & 15u; };
    auto same_page = [](uint32_t a, uint32_t b) { return (a >> 13) == (b >> 13); };
    // the table holds the generic step's key where an instruction would end on its page's last byte (rlenv_hip.hip);
    // a jump to itself is found at run time (fx compares with the CPU address)
    auto generic = [&](uint32_t o) {
        return (o & 0x1FFFu) + len_of(o) >= 0x2000u ||
               jit_always_generic(0xFFFFFFFFu, rd(o), rd(o + 1u), rd(o + 2u), board);
    };
    auto target_of = [&](uint32_t o) { return o + 2u + (uint32_t)(int32_t)(int8_t)rd(o + 1u); };
    std::vector<int> order(size, -1);   // discovery rank of each leader
    std::vector<uint32_t> leaders, work;
    std::vector<char> seen(size, 0), window(0x2000, 0);
    auto entry = [&](uint32_t o) {
        if (o < size && order[o] < 0) {
            order[o] = (int)leaders.size();
            leaders.push_back(o);
            work.push_back(o);
        }
    };
    auto descend = [&]() {
        while (!work.empty()) {
            uint32_t o = work.back();
            work.pop_back();
            while (o < size && !seen[o]) {
                seen[o] = 1;
                const uint32_t grp = grp_of(o), mode = kOptab.t[rd(o)] & 15u, next = o + len_of(o);
                if (generic(o)) {
                    if (grp != G_ILL && grp != G_BRK && grp != G_JMP && same_page(o, next)) entry(next);
                    break;
                }
                if (jit_ppu_store(rd(o), rd(o + 1u), rd(o + 2u))) {
                    if (same_page(o, next)) entry(next);
                    break;
                }
                if (grp == G_BR) {
                    if (same_page(o, target_of(o))) entry(target_of(o));
                    entry(next);
                    break;
                }
                if (grp == G_JMP || grp == G_JSR) {
                    if (mode == M_ABS && rd16(o + 1u) >= 0x8000u) window[rd16(o + 1u) & 0x1FFFu] = 1;
                    if (grp == G_JSR) entry(next);
                    break;
                }
                if (grp == G_RTS || grp == G_RTI) break;
                o = next;
            }
        }
    };
    for (uint32_t v = 0; v < 3; ++v) {
        const uint32_t vec = rd(size - 6u + 2u * v) | (rd(size - 5u + 2u * v) << 8);
        for (uint32_t pg = pages >= 2 ? pages - 2 : 0; pg < pages; ++pg)
            if (((vec >> 13) & 3u) == (pg & 1u ? 3u : 2u) || pages < 2) entry((pg << 13) | (vec & 0x1FFFu));
    }
    descend();
    std::vector<char> seeded(0x2000, 0);
    for (bool grew = true; grew;) {   // window targets into every page, until no new one appears
        grew = false;
        for (uint32_t w = 0; w < 0x2000u; ++w)
            if (window[w] && !seeded[w]) {
                seeded[w] = 1;
                grew = true;
                for (uint32_t pg = 0; pg < pages; ++pg) entry((pg << 13) | w);
            }
        descend();
    }

    // blocks in discovery order within the cap; a block is a run of one page
    std::vector<int> id_of(size, -1);
    struct Block { uint32_t start; std::vector<uint32_t> ins; uint32_t stop; };
    std::vector<Block> kept;
    JitProgram p;
    for (uint32_t start : leaders) {
        Block b{start, {}, start};
        uint32_t o = start;
        for (;;) {
            if (o >= size || !same_page(o, start) || (o != start && order[o] >= 0) || b.ins.size() == kJitMaxBlock ||
                generic(o))
                break;
            b.ins.push_back(o);
            const uint32_t grp = grp_of(o);
            o += len_of(o);
            if (grp == G_BR || grp == G_JMP || grp == G_JSR || grp == G_RTS || grp == G_RTI) break;
        }
        b.stop = o;
        if (b.ins.empty()) continue;
        if (p.instructions + b.ins.size() > kJitMaxInstructions) break;
        id_of[start] = (int)kept.size();
        p.leader_addr.push_back(start);
        p.instructions += (uint32_t)b.ins.size();
        kept.push_back(std::move(b));
    }
    auto go = [&](uint32_t from, uint32_t o) {
        return o < size && same_page(from, o) && id_of[o] >= 0 && o >= from ? "goto JB_" + std::to_string(id_of[o]) + ";"
                                                                           : std::string("continue;");
    };
    auto operand = [&](uint32_t x) {   // the fetch table's decoded operand word (rlenv_hip.hip fetch_entry, banked)
        const uint32_t mode = kOptab.t[rd(x)] & 15u;
        if (mode == M_IMM || mode == M_ZP || mode == M_ZPX || mode == M_ZPY || mode == M_IZX || mode == M_IZY)
            return rd(x + 1u);
        if (mode == M_REL) return (uint32_t)(int32_t)(int8_t)rd(x + 1u) << 3;
        return rd16(x + 1u);
    };
    char buf[200];
    for (size_t i = 0; i < kept.size(); ++i) {
        const Block& b = kept[i];
        const uint32_t last = b.ins.back(), grp = grp_of(last);
        std::string end;
        bool branch_end = false;
        if (grp == G_BR) {
            // taken to another page, the branch leaves the block as needing the generic step (its JIT_STEP); on its
            // page, taken or not each with its cycle count and next pc as constants, as in the fixed translation
            const uint32_t tgt = target_of(last);
            if (same_page(last, tgt)) {
                const uint32_t cyc = (kOptab.t[rd(last)] >> 4) & 15u;
                const uint32_t cross = (((last + 2u) ^ tgt) & 0xFF00u) ? 1u : 0u;
                snprintf(buf, sizeof buf, "if (br_taken<kOptab.t[0x%02Xu]>(h)) { v -= 0x%Xu; h.pc = 0x%Xu; ", rd(last),
                         ((cyc + 1u + cross) << 14) - 1u, tgt << 3);
                const std::string skip = b.ins.size() == 2u ? jit_poll_skip(rd(b.start), rd16(b.start + 1u), rd(last),
                                                                             tgt == b.start, cyc + 1u + cross)
                                                            : std::string();
                end = buf + skip + go(b.start, tgt);
                snprintf(buf, sizeof buf, " } v -= 0x%Xu; h.pc = 0x%Xu; ", (cyc << 14) - 1u, (last + 2u) << 3);
                end += buf + go(b.start, b.stop);
                branch_end = true;
            } else {
                end = go(b.start, b.stop);
            }
        } else if (grp == G_JMP || grp == G_JSR || grp == G_RTS || grp == G_RTI) {
            end = "continue;";
        } else {
            end = go(b.start, b.stop);
        }
        snprintf(buf, sizeof buf, "case 0x%Xu: JB_%zu: {   // PRG $%05X, %zu instructions\n", kBlockKey + (uint32_t)i,
                 i, b.start, b.ins.size());
        p.cases += buf;
        std::string mx;
        for (uint32_t x : b.ins) {
            snprintf(buf, sizeof buf, "%sjit_maxtake(0x%02Xu)", mx.empty() ? "" : " + ", rd(x));
            mx += buf;
        }
        snprintf(buf, sizeof buf, ") { JIT_ONE(0x%02Xu, 0x%Xu, 0x%Xu) }\n", rd(b.start), b.start << 3,
                 operand(b.start));
        p.cases += "    if (v < " + mx + buf;
        for (size_t j = 0; j + (branch_end ? 1u : 0u) < b.ins.size(); ++j) {
            const uint32_t x = b.ins[j];
            snprintf(buf, sizeof buf, "    JIT_STEP(0x%02Xu, 0x%Xu, 0x%Xu)\n", rd(x), x << 3, operand(x));
            p.cases += buf;
        }
        p.cases += "    " + end + "\n}\n";
    }
    return p;
}

// The source of the kernels a translation is compiled into: the console-frame kernel (emu_kernel.h) with the blocks
// (the header "jit_blocks.inc") in its burst loop, launched as rlenv_hip.hip k_emu_w is: k_emu_jit_draw for decision
// frames the emulator's waves draw themselves, and in a bank translation also k_emu_jit for frames drawn from frame
// banks.
// hiprtc has the HIP runtime and the fixed-width integer types built in, the latter in a namespace of its own.
inline std::string jit_module_source(bool bank, bool banked) {
    const std::string board = banked ? "NES_BOARD_MMC3" : "NES_BOARD_NROM";
    return std::string(
               "using __hip_internal::uint8_t;\nusing __hip_internal::uint16_t;\nusing __hip_internal::uint32_t;\n"
               "using __hip_internal::uint64_t;\nusing __hip_internal::int8_t;\nusing __hip_internal::int16_t;\n"
               "using __hip_internal::int32_t;\nusing __hip_internal::int64_t;\n"
               "#ifndef offsetof\n#define offsetof(t, m) __builtin_offsetof(t, m)\n#endif\n"
               "#define RLENV_JIT_INC \"jit_blocks.inc\"\n#include \"emu_kernel.h\"\n") +
           (bank ? std::string("extern \"C\" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n"
                               "void k_emu_jit(nd::EmuArgs a) { nd::emu_body<") +
                       board + ", true, false>(a); }\nND_EMU_KERNEL_ARGS(k_emu_jit);\n"
                 : std::string()) +
           "extern \"C\" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n"
           "void k_emu_jit_draw(nd::EmuArgs a) { nd::emu_body<" + board + ", false, true>(a); }\n"
           "ND_EMU_KERNEL_ARGS(k_emu_jit_draw);\n";
}

}  // namespace nd
