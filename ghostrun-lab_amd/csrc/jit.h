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
// step (I/O other than $2002 reads and $4016, a jump to itself, an unofficial opcode), at the next leader, or after
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
inline bool jit_always_generic(uint32_t a, uint32_t op, uint32_t b1, uint32_t b2) {
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
    if (rd && wr) return ea >= 0x2000u;
    if (wr) return ea >= 0x2000u && ea != 0x4016u;
    if (rd) return !(ea < 0x2000u || ea >= 0x8000u || ea == 0x4016u || (ea & 0xE007u) == 0x2002u);
    return false;
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
        if (grp == G_BR) {
            snprintf(buf, sizeof buf, "if (h.pc == 0x%Xu) ", (target_of(last) & 0x1FFFFu) << 3);
            end = buf + go(b.start, target_of(last)) + " " + go(b.start, b.stop);
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
        for (uint32_t x : b.ins) {
            snprintf(buf, sizeof buf, "    JIT_STEP(0x%02Xu, 0x%Xu, 0x%Xu)\n", rd(x), x << 3, operand(x));
            p.cases += buf;
        }
        p.cases += "    " + end + "\n}\n";
    }
    return p;
}

// The source of the kernel a translation is compiled into: the console-frame kernel (emu_kernel.h) of the fixed-PRG
// boards with the blocks (the header "jit_blocks.inc") in its burst loop, launched as rlenv_hip.hip k_emu_w is.
// hiprtc has the HIP runtime and the fixed-width integer types built in, the latter in a namespace of its own.
inline std::string jit_module_source(bool bank) {
    return std::string(
               "using __hip_internal::uint8_t;\nusing __hip_internal::uint16_t;\nusing __hip_internal::uint32_t;\n"
               "using __hip_internal::uint64_t;\nusing __hip_internal::int8_t;\nusing __hip_internal::int16_t;\n"
               "using __hip_internal::int32_t;\nusing __hip_internal::int64_t;\n"
               "#ifndef offsetof\n#define offsetof(t, m) __builtin_offsetof(t, m)\n#endif\n"
               "#define RLENV_JIT_INC \"jit_blocks.inc\"\n#include \"emu_kernel.h\"\n"
               "extern \"C\" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8)))\n"
               "void k_emu_jit(nd::EmuArgs a) { nd::emu_body<NES_BOARD_NROM, ") +
           (bank ? "true" : "false") + ">(a); }\n";
}

}  // namespace nd
