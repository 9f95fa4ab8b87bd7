// Host-side check of a compiled gfx950 code object for a known miscompile: a far branch that lands where SCC is live.
//
// A branch too far for the 16-bit offset of s_branch / s_cbranch_* is expanded by the compiler after register
// allocation into s_getpc_b64 s[a:b]; s_add_u32 sa, sa, lo; s_addc_u32 sb, sb, hi; s_setpc_b64 s[a:b]. The two adds
// overwrite SCC. The compiler does not check that SCC is dead at the jump: when the code at the target reads SCC
// (s_cselect, s_cbranch_scc*, s_addc_u32, s_subb_u32, s_cmov*) before writing it, that read sees the jump's carry
// instead of the compare made before the jump, and the program computes a wrong value without any error. Only
// kernels of more than 128 KB of code have such jumps: here, the translated kernels of large banked carts.
//
// jit_far_branch_hazards disassembles the .text section (comgr's instruction disassembler), finds every far jump by
// its four-instruction pattern and follows the code from its target, through branches on both sides, until SCC is
// written (safe), the path ends (s_endpgm, s_setpc_b64) or a step limit is reached; an SCC read first is a hazard.
// Anything it cannot follow counts as a hazard, so a code object it passes is free of the pattern.
#pragma once
#include <amd_comgr/amd_comgr.h>
#include <stdint.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace nd {

struct JitInstr {
    uint64_t addr = 0, size = 0;
    std::string text;              // mnemonic and operands
    bool has_target = false;       // an operand resolved to an absolute address (a branch target)
    uint64_t target = 0;
};

struct JitDisasm {
    const uint8_t* bytes = nullptr;
    uint64_t base = 0, size = 0;
    JitInstr* cur = nullptr;
};

inline uint64_t jit_read_cb(uint64_t from, char* to, uint64_t size, void* user) {
    const JitDisasm& d = *static_cast<JitDisasm*>(user);
    if (from < d.base || from >= d.base + d.size) return 0;
    const uint64_t n = std::min<uint64_t>(size, d.base + d.size - from);
    std::memcpy(to, d.bytes + (from - d.base), n);
    return n;
}
inline void jit_print_cb(const char* instruction, void* user) {
    static_cast<JitDisasm*>(user)->cur->text = instruction;
}
inline void jit_addr_cb(uint64_t address, void* user) {
    JitInstr* in = static_cast<JitDisasm*>(user)->cur;
    in->has_target = true;
    in->target = address;
}

// The .text section of an ELF64 code object: its file offset, size and address. False if there is none.
inline bool jit_text_section(const std::vector<char>& co, uint64_t* off, uint64_t* size, uint64_t* addr) {
    auto rd = [&](uint64_t at, int n) -> uint64_t {
        uint64_t v = 0;
        if (at + (uint64_t)n > co.size()) return 0;
        for (int i = n - 1; i >= 0; --i) v = (v << 8) | (uint8_t)co[at + (uint64_t)i];
        return v;
    };
    if (co.size() < 64 || std::memcmp(co.data(), "\x7f" "ELF", 4) != 0 || co[4] != 2) return false;
    const uint64_t shoff = rd(0x28, 8), shentsize = rd(0x3A, 2), shnum = rd(0x3C, 2), shstrndx = rd(0x3E, 2);
    if (shoff == 0 || shentsize < 64 || shstrndx >= shnum) return false;
    const uint64_t strtab = rd(shoff + shstrndx * shentsize + 0x18, 8);
    for (uint64_t s = 0; s < shnum; ++s) {
        const uint64_t h = shoff + s * shentsize;
        const uint64_t name = strtab + rd(h, 4);
        if (name + 6 > co.size() || std::memcmp(co.data() + name, ".text", 6) != 0) continue;
        *addr = rd(h + 0x10, 8);
        *off = rd(h + 0x18, 8);
        *size = rd(h + 0x20, 8);
        return *off + *size <= co.size();
    }
    return false;
}

// Whether an instruction (mnemonic) reads SCC / writes SCC (the scalar ALU's compares, arithmetic and logic).
inline bool jit_reads_scc(const std::string& m) {
    return m.rfind("s_cselect", 0) == 0 || m.rfind("s_cbranch_scc", 0) == 0 || m == "s_addc_u32" ||
           m == "s_subb_u32" || m.rfind("s_cmov", 0) == 0;
}
inline bool jit_writes_scc(const std::string& m) {
    static const char* const kPrefixes[] = {
        "s_cmp", "s_bitcmp", "s_add_u32", "s_sub_u32", "s_add_i32", "s_sub_i32", "s_addk_", "s_and_", "s_or_",
        "s_xor_", "s_andn2_", "s_orn2_", "s_nand_", "s_nor_", "s_xnor_", "s_not_", "s_lshl_", "s_lshr_", "s_ashr_",
        "s_bfe_", "s_min_", "s_max_", "s_abs_", "s_absdiff_", "s_bcnt", "s_quadmask", "s_wqm", "s_lshl1_add",
        "s_lshl2_add", "s_lshl3_add", "s_lshl4_add"};
    for (const char* p : kPrefixes)
        if (m.rfind(p, 0) == 0) return true;
    return false;
}

// The count of far jumps whose target reads SCC before writing it (0: none), or -1 when the code object cannot be
// disassembled. *far_jumps: the far jumps found; *where: the first hazard's target and instruction.
inline int jit_far_branch_hazards(const std::vector<char>& co, int* far_jumps, std::string* where) {
    *far_jumps = 0;
    uint64_t off = 0, size = 0, base = 0;
    if (!jit_text_section(co, &off, &size, &base)) return -1;
    JitDisasm d;
    d.bytes = reinterpret_cast<const uint8_t*>(co.data()) + off;
    d.base = base;
    d.size = size;
    amd_comgr_disassembly_info_t info;
    if (amd_comgr_create_disassembly_info("amdgcn-amd-amdhsa--gfx950", jit_read_cb, jit_print_cb, jit_addr_cb,
                                          &info) != AMD_COMGR_STATUS_SUCCESS)
        return -1;
    std::vector<JitInstr> ins;
    ins.reserve(size / 6);
    for (uint64_t a = base; a < base + size;) {
        JitInstr in;
        in.addr = a;
        d.cur = &in;
        uint64_t n = 0;
        const amd_comgr_status_t st = amd_comgr_disassemble_instruction(info, a, &d, &n);
        if (n == 0) n = 4;
        in.size = n;
        if (st != AMD_COMGR_STATUS_SUCCESS) in.text = "?";
        ins.push_back(std::move(in));
        a += n;
    }
    amd_comgr_destroy_disassembly_info(info);
    std::unordered_map<uint64_t, size_t> at;
    at.reserve(ins.size() * 2);
    for (size_t i = 0; i < ins.size(); ++i) at[ins[i].addr] = i;
    auto mnem = [&](size_t i) {
        const std::string& t = ins[i].text;
        size_t s = t.find_first_not_of(" \t");
        if (s == std::string::npos) return std::string();
        return t.substr(s, t.find_first_of(" \t", s) - s);
    };
    auto last_operand = [&](size_t i, int64_t* v) {   // the immediate after the last comma
        const std::string& t = ins[i].text;
        const size_t c = t.rfind(',');
        if (c == std::string::npos) return false;
        const char* p = t.c_str() + c + 1;
        char* e = nullptr;
        const long long x = std::strtoll(p, &e, 0);
        if (e == p) return false;
        *v = x;
        return true;
    };
    // Follow from instruction index i: 0 when every path writes SCC before reading it or ends, 1 on a hazard.
    std::string first;
    std::vector<char> seen(ins.size(), 0);
    std::vector<size_t> stack;
    auto follow = [&](size_t start) -> int {
        std::fill(seen.begin(), seen.end(), 0);
        stack.assign(1, start);
        int steps = 0;
        while (!stack.empty()) {
            size_t i = stack.back();
            stack.pop_back();
            for (;;) {
                if (i >= ins.size() || ++steps > 100000) {
                    first = "path leaves the code or is too long";
                    return 1;
                }
                if (seen[i]) break;
                seen[i] = 1;
                const std::string m = mnem(i);
                if (m == "?" || m.empty()) {
                    first = "undecodable instruction";
                    return 1;
                }
                if (jit_reads_scc(m)) {
                    char buf[64];
                    snprintf(buf, sizeof buf, "+0x%llx: ", (unsigned long long)(ins[i].addr - base));
                    first = buf + ins[i].text;
                    return 1;
                }
                if (jit_writes_scc(m) || m == "s_endpgm" || m == "s_setpc_b64" || m == "s_code_end") break;
                if (m.rfind("s_cbranch_", 0) == 0 || m == "s_branch") {
                    if (!ins[i].has_target || !at.count(ins[i].target)) {
                        first = "branch without a known target: " + ins[i].text;
                        return 1;
                    }
                    const size_t t = at[ins[i].target];
                    if (m == "s_branch") {
                        i = t;
                        continue;
                    }
                    stack.push_back(t);   // a conditional branch: both ways
                }
                ++i;
            }
        }
        return 0;
    };
    int hazards = 0;
    for (size_t i = 0; i + 3 < ins.size(); ++i) {
        if (mnem(i) != "s_getpc_b64" || mnem(i + 1) != "s_add_u32" || mnem(i + 2) != "s_addc_u32" ||
            mnem(i + 3) != "s_setpc_b64")
            continue;
        int64_t lo = 0, hi = 0;
        if (!last_operand(i + 1, &lo) || !last_operand(i + 2, &hi)) {
            ++hazards;
            if (where->empty()) *where = "far jump with an unreadable offset: " + ins[i + 1].text;
            continue;
        }
        ++*far_jumps;
        const uint64_t target = ins[i].addr + 4u + (((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
        auto it = at.find(target);
        if (it == at.end()) {
            ++hazards;
            if (where->empty()) *where = "far jump to no instruction";
            continue;
        }
        if (follow(it->second)) {
            ++hazards;
            if (where->empty()) {
                char buf[96];
                snprintf(buf, sizeof buf, "far jump at +0x%llx to +0x%llx, then ", (unsigned long long)(ins[i].addr - base),
                         (unsigned long long)(target - base));
                *where = buf + first;
            }
        }
    }
    return hazards;
}

}  // namespace nd
