// Device row layouts of the quantized weights (shared by upload, dequantization and the GEMVs).
//
// Every row starts at row * pitch (pitch a multiple of 16) and is split into planes; inside the
// 4/6-bit quant plane the 16-byte chunks of each pass of 16 super-blocks are permuted so that a
// wave streaming the row reads contiguous bytes AND lane l of the wave gets the two chunks that
// share one 64-element group (q4_K/q5_K) or one set of high bits and scales (q6_K):
//
//   pass P = sb / 16 covers super-blocks 16P .. 16P + m - 1, m = min(16, nsb - 16P);
//   lane l = 4 * (sb % 16) + q takes chunks 128P + l and 128P + 4m + l.
//
// q4_K  : qs[nsb*128] (permuted) | hdr[nsb][16]  (hdr = f16 d, f16 dmin, scales[12])
//         original qs chunk c of a block (bytes 16c..16c+15): q = c/2 (64-element group), e = c%2
// q5_K  : qs[nsb*128] (permuted as q4_K) | qh[nsb][32] | hdr[nsb][16]
// q6_K  : ql[nsb*128] (permuted) | qh[nsb][64] | sc[nsb][16] (permuted) | d[nsb] (f16)
//         original ql chunk c = 4h + 2p + hf (half h, segment parity p, lane half hf):
//         q = 2h + hf, e = p; the sc bytes of a block are regrouped so that dword q holds
//         sc[8h+hf], sc[8h+hf+2], sc[8h+hf+4], sc[8h+hf+6]
// q8_0  : qs[nb][32] | d[nb] (f16)
#pragma once

#include <stdint.h>

namespace oq {

// position, in 16-byte units within the quant plane, of chunk (q, e) of super-block sb
__host__ __device__ inline uint64_t perm_chunk(uint64_t nsb, uint64_t sb, uint32_t q, uint32_t e) {
    const uint64_t pass = sb / 16, s = sb % 16;
    const uint64_t m = nsb - 16 * pass < 16 ? nsb - 16 * pass : 16;
    return 128 * pass + e * 4 * m + 4 * s + q;
}

// byte offset in the q4_K / q5_K quant plane of original qs byte b (0..127) of block sb
__host__ __device__ inline uint64_t q45_qs_offset(uint64_t nsb, uint64_t sb, uint32_t b) {
    const uint32_t c = b / 16;
    return 16 * perm_chunk(nsb, sb, c / 2, c % 2) + (b % 16);
}

// byte offset in the q6_K ql plane of original ql byte b (0..127) of block sb
__host__ __device__ inline uint64_t q6_ql_offset(uint64_t nsb, uint64_t sb, uint32_t b) {
    const uint32_t c = b / 16, h = c / 4, p = (c / 2) % 2, hf = c % 2;
    return 16 * perm_chunk(nsb, sb, 2 * h + hf, p) + (b % 16);
}

// byte offset within a block's 16 regrouped q6_K scales of original scale j (0..15)
__host__ __device__ inline uint32_t q6_sc_offset(uint32_t j) {
    const uint32_t h = j / 8, hf = j % 2, i = (j % 8) / 2;
    return 4 * (2 * h + hf) + i;
}

}  // namespace oq
