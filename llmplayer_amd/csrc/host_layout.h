// Host-side layout arithmetic of the library, in plain C++ with no HIP dependency so that the
// same code also builds with g++ under AddressSanitizer / UndefinedBehaviorSanitizer for the
// CPU tests:
//  - the decode step plan (window start, attended rows, rows per split), shared with the kernels;
//  - the default split count of a decode call;
//  - GGUF row sizes and the repacking of GGUF rows into the per-row planes the projection
//    kernels read;
//  - the re-layout between the reference's row-major KV arrays [pos][n_kv_heads * row] and the
//    head-major staging the device planes use [n_kv_heads][pos][row].
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <vector>

#include "llmp_hip.h"

#ifdef __HIPCC__
#define LLMP_HD __host__ __device__
#else
#define LLMP_HD
#endif

namespace llmp {

// Step plan shared by host and kernels: window start, attended rows, rows per split (rounded
// to 16 once there are at least 16 per split) and the splits that end up non-empty.
struct StepPlan {
    int start, n, rows_per_split, splits;
};
LLMP_HD inline StepPlan plan_step(int pos, int window, int max_splits) {
    StepPlan p;
    p.start = (window > 0 && pos - window + 1 > 0) ? pos - window + 1 : 0;
    p.n = pos + 1 - p.start;
    int s = max_splits < p.n ? max_splits : p.n;
    if (s < 1) s = 1;
    int rps = (p.n + s - 1) / s;
    if (p.n >= 16 * s) rps = (rps + 15) & ~15;
    p.rows_per_split = rps;
    p.splits = (p.n + rps - 1) / rps;
    return p;
}

// Head shapes the decode kernels are instantiated for: head_dim 64/128/256/512 with GQA groups
// 1-8, 96 with 1-4 (Phi-3) and 80 with 1-2 (Phi-2).
inline bool decode_group_ok(int head_dim, int group) {
    const int limit = (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512)
                          ? 8
                          : (head_dim == 96 ? 4 : (head_dim == 80 ? 2 : 0));
    return group >= 1 && group <= limit;
}
// The group the kernels run a layer with: `group` itself when instantiated, else its largest
// divisor that is (a layer of G query heads per KV head then runs as G / divisor virtual KV heads
// per cached KV head, each with `divisor` query heads); 0 when no divisor is.
inline int kernel_group(int head_dim, int group) {
    if (group < 1) return 0;
    for (int g = group < 8 ? group : 8; g >= 1; --g)
        if (group % g == 0 && decode_group_ok(head_dim, g)) return g;
    return 0;
}

// Default split count of a decode step over n attended rows, given the CUs and the workgroups
// of the chosen kernel resident per CU (per_cu; 1 for fp32 caches, which aim at one workgroup
// per CU):
//  - fp32: at least 32 rows per split (16 where 32-row splits of all KV heads would not cover
//    half of the CUs: few KV heads over a short window), at most 128 splits per KV head; once a
//    split holds 1024 rows or more, `wide` is set (8-wave workgroups) and 3/4 of the splits run.
//  - Q8_0: one full round of resident workgroups over the chip, at least 160 rows per split.
inline int default_splits(int n, int n_kv_heads, int n_cu, int per_cu, bool q8, bool* wide) {
    const int cu = n_cu > 0 ? n_cu : 256;
    int min_rows = q8 ? 160 : 32;
    if (!q8 && 2LL * n_kv_heads * (n / 32) < cu) min_rows = 16;
    const int by_rows = n / min_rows > 0 ? n / min_rows : 1;
    if (per_cu < 1) per_cu = 1;
    long long s = ((long long)per_cu * cu + n_kv_heads - 1) / n_kv_heads;
    if (s > by_rows) s = by_rows;
    if (s > 128) s = 128;
    if (s < 1) s = 1;
    *wide = false;
    if (!q8 && n / s >= 1024) {
        *wide = true;
        s = (3 * s + 3) / 4;
    }
    return (int)s;
}

// Workgroups per query head of the split combine (column groups of the head's D values): the
// fewest of 1, 2, 4, 8 with which each of the `threads` threads of a group holds at most `batch`
// of the `splits` partials (all its loads in one round), keeping whole float4 columns and at
// least 4 of them per group.
inline int reduce_column_groups(int D, int splits, int threads, int batch) {
    const int nc = D / 4;
    int cb = 1;
    while (cb < 8 && nc % (2 * cb) == 0 && nc / (2 * cb) >= 4 &&
           (long long)splits > (long long)batch * (threads / (nc / cb)))
        cb *= 2;
    return cb;
}

// Bytes of one row of `cols` weights in a GGML type's GGUF layout (GGMLType.java:4-35); 0 for
// a type the library does not read.
inline size_t ggml_row_bytes(int type, int cols) {
    switch (type) {
    case LLMP_GGML_F32: return (size_t)cols * 4;
    case LLMP_GGML_F16:
    case LLMP_GGML_BF16: return (size_t)cols * 2;
    case LLMP_GGML_Q8_0: return (size_t)(cols / 32) * 34;
    case LLMP_GGML_Q4_0: return (size_t)(cols / 32) * 18;
    case LLMP_GGML_Q4_K: return (size_t)(cols / 256) * 144;
    case LLMP_GGML_Q6_K: return (size_t)(cols / 256) * 210;
    case LLMP_GGML_Q5_0: return (size_t)(cols / 32) * 22;
    case LLMP_GGML_Q3_K: return (size_t)(cols / 256) * 110;
    case LLMP_GGML_Q5_K: return (size_t)(cols / 256) * 176;
    case LLMP_GGML_IQ4_NL: return (size_t)(cols / 32) * 18;
    case LLMP_GGML_IQ4_XS: return (size_t)(cols / 256) * 136;
    case LLMP_GGML_MXFP4: return (size_t)(cols / 32) * 17;
    case LLMP_GGML_Q5_1: return (size_t)(cols / 32) * 24;
    case LLMP_GGML_Q2_K: return (size_t)(cols / 256) * 84;
    case LLMP_GGML_IQ3_XXS: return (size_t)(cols / 256) * 98;
    case LLMP_GGML_IQ3_S: return (size_t)(cols / 256) * 110;
    case LLMP_GGML_IQ2_S: return (size_t)(cols / 256) * 82;
    default: return 0;
    }
}

// Q3_K's 16 six-bit sub-block scales from the 12 packed bytes at offset 96 of a super-block
// (Q3_KFloatTensor.decodeAllScales, Q3_KFloatTensor.java:128-143): scale k has its low four
// bits in byte k%8 (low nibble for k < 8, high nibble after) and its top two bits at bits
// 2(k/4)..+1 of byte 8 + k%4.  Stored as the int8 sc - 32, the factor d multiplies.
inline void q3k_scales(const uint8_t* raw, int8_t out[16]) {
    for (int k = 0; k < 16; ++k) {
        const int low = k < 8 ? (raw[k] & 15) : (raw[k - 8] >> 4);
        const int top = (raw[8 + k % 4] >> (2 * (k / 4))) & 3;
        out[k] = (int8_t)((low | (top << 4)) - 32);
    }
}
// IQ4_XS's 8 six-bit sub-block scales from bytes 2..7 of a super-block (IQ4_XSFloatTensor.dot,
// IQ4_XSFloatTensor.java:63-69): low four bits from scales_l (byte 4 + ib/2, low nibble for
// even ib), top two bits from scales_h (uint16 at byte 2, bits 2ib..2ib+1); stored as ls - 32.
inline void iq4xs_scales(const uint8_t* blk, int8_t out[8]) {
    const int sh = blk[2] | (blk[3] << 8);
    for (int ib = 0; ib < 8; ++ib) {
        const int sl = blk[4 + ib / 2];
        const int low = (ib & 1) ? (sl >> 4) : (sl & 15);
        out[ib] = (int8_t)((low | (((sh >> (2 * ib)) & 3) << 4)) - 32);
    }
}

// IQ3_XXS's per-32-group words (bytes 66 + 4 ib32 of a super-block, little-endian; the
// IQ3_XXSFloatTensor.dot fields): the four 7-bit sign-pattern indices at bits 7l expanded to
// the 8-bit patterns (KSIGNS_IQ2XS: the eighth bit makes the count of set bits even) -> signs
// [32] (8-weight group 4 ib32 + l), and the 4-bit scales at bits 28-31 -> nibble ib32%2 of
// scales[ib32/2].
inline void iq3xxs_signs_scales(const uint8_t* blk, uint8_t signs[32], uint8_t scales[4]) {
    for (int i = 0; i < 4; ++i) scales[i] = 0;
    for (int ib = 0; ib < 8; ++ib) {
        const uint8_t* a = blk + 66 + 4 * ib;
        const uint32_t aux = (uint32_t)a[0] | ((uint32_t)a[1] << 8) | ((uint32_t)a[2] << 16) | ((uint32_t)a[3] << 24);
        for (int l = 0; l < 4; ++l) {
            const uint32_t i7 = (aux >> (7 * l)) & 0x7Fu;
            uint32_t par = 0;
            for (int k = 0; k < 7; ++k) par ^= (i7 >> k) & 1u;
            signs[4 * ib + l] = (uint8_t)(i7 | (par << 7));
        }
        scales[ib / 2] = (uint8_t)(scales[ib / 2] | ((aux >> 28) << (4 * (ib & 1))));
    }
}

inline size_t pad256(size_t b) { return (b + 255) & ~(size_t)255; }

// Range exponent of a stored value, as the kernels' dk::range_exp_of_bits computes it:
// max(0, floor(log2|x|) - 14), 0 for |x| < 2^15, so that |x| * 2^-E < 2^15 (the fp16 hi/lo
// split of the multi-token kernels needs magnitudes below 65504).
inline int range_exp(float x) {
    uint32_t b;
    std::memcpy(&b, &x, sizeof b);
    const int e = (int)((b & 0x7FFFFFFFu) >> 23) - 141;
    return e > 0 ? e : 0;
}
// Raises ek[h] / ev[h] (h < H) to the range exponents of n rows in the reference layout
// [t][H * row] (row values per KV head); k or v may be null.
inline void range_exp_rows(const float* k, const float* v, size_t H, size_t n, size_t row, int* ek,
                           int* ev) {
    for (size_t t = 0; t < n; ++t)
        for (size_t h = 0; h < H; ++h)
            for (size_t j = 0; j < row; ++j) {
                const size_t i = (t * H + h) * row + j;
                if (k) { const int e = range_exp(k[i]); if (e > ek[h]) ek[h] = e; }
                if (v) { const int e = range_exp(v[i]); if (e > ev[h]) ev[h] = e; }
            }
}
// The same for Q8_0 rows (quants [t][H * row], scales [t][H * row / 32]), over the values the
// kernels dequantise: (float)quant * scale.
inline void range_exp_rows_q8(const int8_t* q, const float* s, size_t H, size_t n, size_t row,
                              int* e_out) {
    for (size_t t = 0; t < n; ++t)
        for (size_t h = 0; h < H; ++h)
            for (size_t j = 0; j < row; ++j) {
                const size_t i = (t * H + h) * row + j;
                const int e = range_exp((float)q[i] * s[i / 32]);
                if (e > e_out[h]) e_out[h] = e;
            }
}

// Repacks `rows` GGUF rows of `cols` weights (src, ggml_row_bytes(type, cols) bytes each) into
// the planes the projection kernels read: every row's bytes of one plane are contiguous
// (pitch[i] bytes per row) and each plane starts 256-byte aligned at off[i] in dst.  Per GGUF
// block the pieces go to:
//  - Q8_0: quants -> plane 0, fp16 scale -> plane 1;
//  - Q4_0: nibbles -> plane 0, fp16 scale -> plane 1;
//  - Q4_K: d, dmin and the 12 packed scale bytes -> plane 1, nibbles -> plane 0;
//  - Q6_K: low nibbles -> 0, high bit pairs -> 1, int8 scales -> 2, fp16 d -> 3;
//  - Q5_0: nibbles -> 0, the 32 fifth bits (uint32) -> 1, fp16 scale -> 2;
//  - Q3_K: 2-bit quants -> 0, high-bit mask -> 1, the 16 scales decoded to int8 sc - 32 -> 2,
//    fp16 d -> 3;
//  - Q5_K: nibbles -> 0, d, dmin and the 12 packed scale bytes -> 1, fifth bits -> 2;
//  - IQ4_NL: nibble codes -> 0, fp16 scale -> 1;
//  - IQ4_XS: nibble codes -> 0, the 8 scales decoded to int8 ls - 32 -> 1, fp16 d -> 2;
//  - MXFP4: nibble codes -> 0, E8M0 exponent byte -> 1;
//  - Q5_1: nibbles -> 0, the 32 fifth bits (uint32) -> 1, fp16 d -> 2, fp16 m -> 3;
//  - Q2_K: the 64 quant bytes -> 0, the 16 scale/min bytes -> 1, fp16 d -> 2, fp16 dmin -> 3;
//  - IQ3_XXS: the 64 codebook indices -> 0, the 32 sign patterns expanded to bytes -> 1,
//    per super-block 8 bytes -> 2: fp16 d, 2 pad, the eight 4-bit scales;
//  - IQ3_S: qs (64) -> 0, signs (32) -> 1, per super-block 16 bytes -> 2: qh[8], scales[4],
//    fp16 d, 2 pad;
//  - IQ2_S: qs (32) -> 0, signs (32) -> 1, per super-block 24 bytes -> 2: scales[8], qh[8],
//    fp16 d, 6 pad;
//  - F32/F16/BF16: one plane, the rows unchanged.
// Returns the plane count, or 0 for an unsupported type or a cols that is not a whole number
// of blocks.
inline int repack_weight(int type, int rows, int cols, const uint8_t* src, std::vector<uint8_t>& dst,
                         size_t off[4], size_t pitch[4]) {
    const size_t rb = ggml_row_bytes(type, cols);
    if (rb == 0 || rows < 0 || cols <= 0) return 0;
    int n = 1;
    // per block: bytes [src_off, +len) -> plane, at dst_off in the block's pitch/blocks bytes
    struct Piece { int plane; size_t src_off, len, dst_off; };
    Piece pieces[6];
    int n_pieces = 0;
    size_t bw = 0, blk_bytes = 0;   // weights and bytes per GGUF block
    auto set = [&](std::initializer_list<Piece> l) {
        for (const Piece& p : l) pieces[n_pieces++] = p;
    };
    switch (type) {
    case LLMP_GGML_F32: case LLMP_GGML_F16: case LLMP_GGML_BF16:
        pitch[0] = rb; break;
    case LLMP_GGML_Q8_0:
        n = 2; bw = 32; blk_bytes = 34; pitch[0] = (size_t)cols; pitch[1] = (size_t)cols / 32 * 2;
        set({{1, 0, 2}, {0, 2, 32}}); break;
    case LLMP_GGML_Q4_0:
        n = 2; bw = 32; blk_bytes = 18; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 32 * 2;
        set({{1, 0, 2}, {0, 2, 16}}); break;
    case LLMP_GGML_Q4_K:
        n = 2; bw = 256; blk_bytes = 144; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 256 * 16;
        set({{1, 0, 16}, {0, 16, 128}}); break;
    case LLMP_GGML_Q6_K:
        n = 4; bw = 256; blk_bytes = 210; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 4;
        pitch[2] = (size_t)cols / 16; pitch[3] = (size_t)cols / 256 * 2;
        set({{0, 0, 128}, {1, 128, 64}, {2, 192, 16}, {3, 208, 2}}); break;
    case LLMP_GGML_Q5_0:
        n = 3; bw = 32; blk_bytes = 22; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 32 * 4;
        pitch[2] = (size_t)cols / 32 * 2;
        set({{2, 0, 2}, {1, 2, 4}, {0, 6, 16}}); break;
    case LLMP_GGML_Q3_K:   // plane 2 (decoded scales) is written below
        n = 4; bw = 256; blk_bytes = 110; pitch[0] = (size_t)cols / 4; pitch[1] = (size_t)cols / 8;
        pitch[2] = (size_t)cols / 16; pitch[3] = (size_t)cols / 256 * 2;
        set({{1, 0, 32}, {0, 32, 64}, {3, 108, 2}}); break;
    case LLMP_GGML_Q5_K:
        n = 3; bw = 256; blk_bytes = 176; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 256 * 16;
        pitch[2] = (size_t)cols / 8;
        set({{1, 0, 16}, {2, 16, 32}, {0, 48, 128}}); break;
    case LLMP_GGML_IQ4_NL:
        n = 2; bw = 32; blk_bytes = 18; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 32 * 2;
        set({{1, 0, 2}, {0, 2, 16}}); break;
    case LLMP_GGML_IQ4_XS:   // plane 1 (decoded scales) is written below
        n = 3; bw = 256; blk_bytes = 136; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 32;
        pitch[2] = (size_t)cols / 256 * 2;
        set({{2, 0, 2}, {0, 8, 128}}); break;
    case LLMP_GGML_MXFP4:
        n = 2; bw = 32; blk_bytes = 17; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 32;
        set({{1, 0, 1}, {0, 1, 16}}); break;
    case LLMP_GGML_Q5_1:
        n = 4; bw = 32; blk_bytes = 24; pitch[0] = (size_t)cols / 2; pitch[1] = (size_t)cols / 32 * 4;
        pitch[2] = pitch[3] = (size_t)cols / 32 * 2;
        set({{2, 0, 2}, {3, 2, 2}, {1, 4, 4}, {0, 8, 16}}); break;
    case LLMP_GGML_Q2_K:
        n = 4; bw = 256; blk_bytes = 84; pitch[0] = (size_t)cols / 4; pitch[1] = (size_t)cols / 16;
        pitch[2] = pitch[3] = (size_t)cols / 256 * 2;
        set({{1, 0, 16}, {0, 16, 64}, {2, 80, 2}, {3, 82, 2}}); break;
    case LLMP_GGML_IQ3_XXS:   // plane 1 and the scales of plane 2 are written below
        n = 3; bw = 256; blk_bytes = 98; pitch[0] = (size_t)cols / 4; pitch[1] = (size_t)cols / 8;
        pitch[2] = (size_t)cols / 256 * 8;
        set({{0, 2, 64}, {2, 0, 2}}); break;
    case LLMP_GGML_IQ3_S:
        n = 3; bw = 256; blk_bytes = 110; pitch[0] = (size_t)cols / 4; pitch[1] = (size_t)cols / 8;
        pitch[2] = (size_t)cols / 256 * 16;
        set({{0, 2, 64}, {1, 74, 32}, {2, 66, 8, 0}, {2, 106, 4, 8}, {2, 0, 2, 12}}); break;
    case LLMP_GGML_IQ2_S:
        n = 3; bw = 256; blk_bytes = 82; pitch[0] = (size_t)cols / 8; pitch[1] = (size_t)cols / 8;
        pitch[2] = (size_t)cols / 256 * 24;
        set({{0, 2, 32}, {1, 34, 32}, {2, 74, 8, 0}, {2, 66, 8, 8}, {2, 0, 2, 16}}); break;
    default: return 0;
    }
    if (bw && cols % (int)bw) return 0;
    off[0] = 0;
    for (int i = 1; i < n; ++i) off[i] = pad256(off[i - 1] + (size_t)rows * pitch[i - 1]);
    dst.assign(pad256(off[n - 1] + (size_t)rows * pitch[n - 1]), 0);
    if (n_pieces == 0) {
        for (int r = 0; r < rows; ++r) std::memcpy(&dst[(size_t)r * pitch[0]], src + (size_t)r * rb, rb);
        return n;
    }
    const size_t nb = (size_t)cols / bw;
    for (int r = 0; r < rows; ++r)
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t* blk = src + (size_t)r * rb + b * blk_bytes;
            for (int i = 0; i < n_pieces; ++i) {
                const Piece& pc = pieces[i];
                std::memcpy(&dst[off[pc.plane] + (size_t)r * pitch[pc.plane] + b * (pitch[pc.plane] / nb) + pc.dst_off],
                            blk + pc.src_off, pc.len);
            }
            if (type == LLMP_GGML_Q3_K)
                q3k_scales(blk + 96, reinterpret_cast<int8_t*>(&dst[off[2] + (size_t)r * pitch[2] + b * 16]));
            else if (type == LLMP_GGML_IQ4_XS)
                iq4xs_scales(blk, reinterpret_cast<int8_t*>(&dst[off[1] + (size_t)r * pitch[1] + b * 8]));
            else if (type == LLMP_GGML_IQ3_XXS)
                iq3xxs_signs_scales(blk, &dst[off[1] + (size_t)r * pitch[1] + b * 32],
                                    &dst[off[2] + (size_t)r * pitch[2] + b * 8 + 4]);
        }
    return n;
}

// Re-layout between n rows of the reference's KV arrays, host[t][h * row + j] (t < n, h < H,
// j < row bytes), and the head-major staging stage[h][t][row], in which each KV head's n rows
// are one contiguous span of n * row bytes.
inline void rows_to_heads(const void* host, void* stage, size_t H, size_t n, size_t row) {
    const char* hp = static_cast<const char*>(host);
    char* sp = static_cast<char*>(stage);
    const size_t span = row * n, host_row = row * H;
    for (size_t t = 0; t < n; ++t)
        for (size_t h = 0; h < H; ++h) std::memcpy(sp + h * span + t * row, hp + t * host_row + h * row, row);
}
inline void heads_to_rows(const void* stage, void* host, size_t H, size_t n, size_t row) {
    const char* sp = static_cast<const char*>(stage);
    char* hp = static_cast<char*>(host);
    const size_t span = row * n, host_row = row * H;
    for (size_t t = 0; t < n; ++t)
        for (size_t h = 0; h < H; ++h) std::memcpy(hp + t * host_row + h * row, sp + h * span + t * row, row);
}

}  // namespace llmp
