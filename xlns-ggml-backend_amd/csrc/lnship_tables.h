// Arithmetic tables of the xlns16 / xlns32 formats, built on the host once
// and copied to every device (the reference copies xlnscpp's host tables the
// same way, lns-backend/cuda/lns-cuda-xlns16.cu:132-140).
#pragma once

#include <cstdint>

namespace lnship {

// xlns16: sign bit 15, log field 128*log2|x| + 0x4000 in bits 14..0.
constexpr uint32_t k16_sign = 0x8000u, k16_logmask = 0x7fffu, k16_one = 0x4000u;
constexpr int k16_esszer = 1280;          // addends further than this are dropped
constexpr int k16_gauss_n = k16_esszer + 2;  // entries per Gaussian-log table
// Monte addition: the base Gaussian log below k16_mc_start; from there a draw
// of one ulp with probability F(d)/64, F(d) = floor(2^(-d/128) * 185 * 64),
// which is 0 from k16_mc_end on
constexpr int k16_mc_start = 1091, k16_mc_end = 1732;
constexpr int k16_mc_n = k16_mc_end + 1;   // entries per Monte table

// xlns32: sign bit 31, log field 2^23*log2|x| + 0x40000000.
constexpr uint32_t k32_sign = 0x80000000u, k32_logmask = 0x7fffffffu, k32_one = 0x40000000u;
constexpr uint32_t k32_esszer = 24u << 23;
// sb grid: 2^13 below 12 binades, 2^19 from 12 to 24 binades
constexpr uint32_t k32_sb_end = 12u << 23;
constexpr int k32_sb_sh = 13, k32_sb_fsh = 19;
constexpr int k32_sb_n = (int)(k32_sb_end >> k32_sb_sh) + 1;                   // 12289
constexpr int k32_sb_fn = (int)((k32_esszer - k32_sb_end) >> k32_sb_fsh) + 1;  // 193
// db grid: cotransformation below 2 binades, 2^13 from 2 to 8, 2^19 to 24
constexpr uint32_t k32_co_end = 1u << 24;
constexpr int k32_co_sh = 12;
constexpr int k32_co_n = 1 << k32_co_sh;                                       // 4096 each
constexpr uint32_t k32_db_end = 8u << 23;
constexpr int k32_db_sh = 13, k32_db_fsh = 19;
constexpr int k32_db_first = (int)(k32_co_end >> k32_db_sh);                   // 2048
constexpr int k32_db_n = (int)(k32_db_end >> k32_db_sh) + 1 - k32_db_first;    // 6145
constexpr int k32_db_fn = (int)((k32_esszer - k32_db_end) >> k32_db_fsh) + 1;  // 257

// One contiguous int32 block for the xlns32 adder, in this order (the
// cotransformation tables first: their LDS byte offsets fit in the 16-bit
// immediate of an LDS read).
constexpr int k32_off_dlo = 0;
constexpr int k32_off_dhi = k32_off_dlo + k32_co_n;
constexpr int k32_off_sb = k32_off_dhi + k32_co_n;
constexpr int k32_off_sbf = k32_off_sb + k32_sb_n;
constexpr int k32_off_db = k32_off_sbf + k32_sb_fn;
constexpr int k32_off_dbf = k32_off_db + k32_db_n;
constexpr int k32_tab_n = k32_off_dbf + k32_db_fn;                             // 27076

constexpr int k_lp_n = 256;   // entries of each lpvip db table

struct host_tables {
    uint16_t cvt16[1u << 17];   // float bits >> 15 -> xlns16
    float    rev16[1u << 16];   // xlns16 -> float
    int16_t  gauss16[2 * k16_gauss_n];   // [0]: sb, [1]: db at distance d; d = esszer + 1 -> 0
    // Monte, per distance d < k16_mc_n: (sb e, sb m, db e, db m); the
    // adjustment is (e + ((r ^ (m >> 31)) & m)) >> 6 with r the top 6 bits of
    // the new LFSR state: (64 table, 0) below the dither range, then sb
    // (F(d), 63) = +((F + r) >> 6) and db (64 - F(d), -1) = -((F + r) >> 6)
    int32_t  gauss16m[4 * k16_mc_n];
    uint16_t exp16[1u << 16];   // xlns16 -> xlns16 exp
    uint16_t sig16[1u << 16];   // xlns16 -> xlns16 sigmoid (silu = x * sigmoid)
    int32_t  tab32[k32_tab_n];  // xlns32 adder tables, layout above
    uint16_t lfsr_seq[65536];   // LFSR state after i steps from state 1 (i < 65535)
    uint16_t lfsr_log[65536];   // inverse of lfsr_seq
    // lpvip's Gaussian log for opposite signs below one binade, evaluated
    // from tables: 2^(-k/256), 1/(1 + j/256) and log2(1 + j/256), k, j < 256
    double lpdb[3 * k_lp_n];
};

// Fills t (a ~1.1 MB object); deterministic.
void build_host_tables(host_tables &t);

}  // namespace lnship
