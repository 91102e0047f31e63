// common.h -- device helpers shared by the gfx950 kernels of libchimere_hip.
//
// Arithmetic contract: every kernel is compiled with -ffp-contract=off; a
// fused multiply-add appears only where written as __builtin_fmaf.  Float
// division is IEEE (hipcc's default correctly rounded divide).  Together with
// det_exp() below this makes every fp32 result reproducible bit for bit by a
// CPU restatement that performs the same operations in the same order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq3s_grid.inc"

namespace chimere {

// ggml type ids
enum : int { T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ3_S = 21, T_MXFP4 = 39 };
// Internal id, not a ggml type: Q4_0 blocks with ggml's block term
// d_w * (sum(nib * q_x) * d_x - 8 * s_x) (the "s-form", s_x = the Q8_1 block's
// f16 sum of x) instead of the exact integer form; chimere_mmvq_q4_0_sform only.
constexpr int T_Q4_0S = 102;

constexpr int QK = 32;             // elements per Q8_0 / Q4_0 / Q8_1 block
constexpr int Q8_1_BYTES = 36;     // [f16 d][f16 s][i8 q[32]]
constexpr int ROW_PAD = 512;       // ggml MATRIX_ROW_PADDING
constexpr int SLOTS = 16;          // lanes per row in the GEMV kernels (the L of the fp32 order)
constexpr int TILE_ROWS = 16;      // rows per GEMV work-group tile (one per 16-lane group)
constexpr int GEMV_THREADS = TILE_ROWS * SLOTS;   // 256 = 4 waves of 64
constexpr int CHUNK_BLOCKS = 64;   // 32-element blocks of one row held in LDS at a time

// IQ3_S codebook with the block's sign bits folded in: entry 16 * i + n is
// codebook entry i with byte k negated where bit k of the 4-bit nibble n is
// set, so one lookup gives four signed int8 levels (8192 words, 32 KiB of
// LDS, against 512 words and per-word sign masks).  Generated at compile
// time from the codebook.
struct Iq3sSignedGrid {
    uint32_t w[8192];
    constexpr Iq3sSignedGrid() : w() {
        constexpr uint32_t base[512] = CHIMERE_IQ3S_GRID_INIT;
        for (int i = 0; i < 512; i++)
            for (int n = 0; n < 16; n++) {
                uint32_t v = 0;
                for (int k = 0; k < 4; k++) {
                    const uint32_t b = (base[i] >> (8 * k)) & 0xFFu;
                    v |= (((n >> k) & 1) ? ((0x100u - b) & 0xFFu) : b) << (8 * k);
                }
                w[16 * i + n] = v;
            }
    }
};
static __device__ const Iq3sSignedGrid c_iq3s_sgrid{};
// Fills a work-group's LDS copy of the sign-folded codebook (8192 words, 16-byte
// aligned); the caller synchronises before use.
__device__ __forceinline__ void iq3s_sgrid_fill(uint32_t* lds, int tid, int nth) {
    const uint4* src = (const uint4*)c_iq3s_sgrid.w;
    for (int i = tid; i < 2048; i += nth) ((uint4*)lds)[i] = src[i];
}

__host__ __device__ inline int64_t pad_to(int64_t n, int64_t a) { return (n + a - 1) / a * a; }

template <int T> struct QTraits;
template <> struct QTraits<T_Q8_0>  { static constexpr int BYTES = 34;  static constexpr int ELEMS = 32; };
template <> struct QTraits<T_Q4_0>  { static constexpr int BYTES = 18;  static constexpr int ELEMS = 32; };
template <> struct QTraits<T_Q4_0S> { static constexpr int BYTES = 18;  static constexpr int ELEMS = 32; };
template <> struct QTraits<T_IQ3_S> { static constexpr int BYTES = 110; static constexpr int ELEMS = 256; };
template <> struct QTraits<T_Q4_K>  { static constexpr int BYTES = 144; static constexpr int ELEMS = 256; };
template <> struct QTraits<T_Q5_K>  { static constexpr int BYTES = 176; static constexpr int ELEMS = 256; };
template <> struct QTraits<T_Q6_K>  { static constexpr int BYTES = 210; static constexpr int ELEMS = 256; };
template <> struct QTraits<T_MXFP4> { static constexpr int BYTES = 17;  static constexpr int ELEMS = 32; };

// Block bytes / elements per block of a type id (0 for an unknown type).
__host__ __device__ inline int type_block_bytes(int type) {
    switch (type) {
    case T_Q8_0: return 34;
    case T_Q4_0: return 18;
    case T_IQ3_S: return 110;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    case T_MXFP4: return 17;
    default: return 0;
    }
}
__host__ __device__ inline int type_block_elems(int type) {
    return type == T_IQ3_S || type == T_Q4_K || type == T_Q5_K || type == T_Q6_K ? 256 : 32;
}
__host__ __device__ inline int64_t row_bytes(int type, int64_t ncols) {
    return ncols / type_block_elems(type) * type_block_bytes(type);
}

__device__ __forceinline__ float h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f2h(float x) {   // round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// Deterministic exp (same operation sequence as the CPU oracle): Cody-Waite
// reduction with ln2 split 0x1.62e4p-1 + 0x1.7f7d1cp-20, degree-7 Taylor
// polynomial of e^r in Horner form, scaling by 2^n.  x < -86 -> 0,
// x > 88.7228 -> +inf.  Relative error about 1 ulp.
// Branch-free: the polynomial runs on x clamped to the finite range and the
// special cases are selected afterwards (identical results, and several
// exponentials in a row interleave).
__device__ __forceinline__ float det_exp(float x) {
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -86.0f), 88.72283905f);
    float n = __builtin_rintf(xc * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, xc);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float e = __builtin_ldexpf(p, (int)n);
    e = x < -86.0f ? 0.0f : e;
    e = x > 88.72283905f ? __builtin_huge_valf() : e;
    return x != x ? x : e;
}
// silu(g) = g / (1 + exp(-g))   (fused_ops.rs:34-45)
__device__ __forceinline__ float det_silu(float g) { return g / (1.0f + det_exp(-g)); }

__device__ __forceinline__ int dot4(int a, int b, int c) {   // v_dot4_i32_i8
    return __builtin_amdgcn_sdot4(a, b, c, false);
}
// byte i = bit i of the 4-bit nibble (0x00 / 0x01)
__device__ __forceinline__ uint32_t nib_bits(uint32_t nib) {
    return (nib * 0x00204081u) & 0x01010101u;   // 24-bit multiply: nib < 16
}
// bytes 0xFF where the corresponding bit of the 4-bit nibble is set
// (v_perm_b32 selector 12 yields 0x00, 13 yields 0xFF)
__device__ __forceinline__ uint32_t nib_mask(uint32_t nib) {
    return __builtin_amdgcn_perm(0u, 0u, nib_bits(nib) | 0x0C0C0C0Cu);
}
// Sign masks of the two nibbles of byte j of s: bytes 0xFF where bit i (low
// nibble: m0) / bit 4 + i (high nibble: m1) is set, i = byte index.  One
// v_perm replicates the byte; each mask is then one AND and one v_perm whose
// selector byte is 0 (byte 0 of 0xFFFFFF00: 0x00) or 1, 2, 4 (0xFF bytes of
// the sources), 8 (the sign of byte 1 of 0xFFFFFF00: 0xFF) or 16..128
// (>= 13: 0xFF).
__device__ __forceinline__ void byte_sign_masks(uint32_t s, int j, uint32_t& m0, uint32_t& m1) {
    const uint32_t r = __builtin_amdgcn_perm(s, s, 0x01010101u * (uint32_t)j);
    m0 = __builtin_amdgcn_perm(0xFFFFFFFFu, 0xFFFFFF00u, r & 0x08040201u);
    m1 = __builtin_amdgcn_perm(0xFFFFFFFFu, 0xFFFFFF00u, r & 0x80402010u);
}
// (hi:lo) >> 8*s, s in 0..3
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}
// 4 bytes at any byte offset of a 4-byte aligned LDS buffer (needs 4 bytes slack)
__device__ __forceinline__ uint32_t lds_u32(const uint8_t* base, int off) {
    const uint32_t* w = (const uint32_t*)(base + (off & ~3));
    return align_bytes(w[1], w[0], off & 3);
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* base, int off) {
    return *(const uint16_t*)(base + off);   // off is even for every block field read this way
}

// One Q8_1 activation block in registers.
struct XBlk {
    int q[8];
    float d;
    int sumq;        // sum of the 32 quants (used by Q4_0's "- 8" term)
    uint32_t sbits;  // the block's f16 s = sum of x (used by the Q4_0 s-form only)
};

__device__ __forceinline__ void load_xblk(const uint8_t* __restrict__ p, XBlk& x) {
    const uint32_t* w = (const uint32_t*)p;   // 36-byte blocks are 4-byte aligned
    uint32_t w0 = w[0];
    x.d = h2f(w0 & 0xFFFFu);
    x.sbits = w0 >> 16;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) { x.q[i] = (int)w[1 + i]; s = dot4(x.q[i], 0x01010101, s); }
    x.sumq = s;
}

// ---- exact int32 block dots of one weight block with one Q8_1 block.
// The *_core functions take the block's fields already in registers; the
// LDS versions read them at byte offset `off` (IQ3_S: of the 110-byte
// superblock) within `row`.  They return sumi and set *dw = f32(weight scale).

__device__ __forceinline__ int dot_q8_0_core(uint32_t dbits, const uint32_t (&q)[8], const XBlk& x, float* dw) {
    *dw = h2f(dbits);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = dot4((int)q[i], x.q[i], s);
    return s;
}

__device__ __forceinline__ int dot_q4_0_core(uint32_t dbits, const uint32_t (&qs)[4], const XBlk& x, float* dw) {
    *dw = h2f(dbits);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s = dot4((int)(qs[i] & 0x0F0F0F0Fu), x.q[i], s);          // elements 4i..4i+3
        s = dot4((int)((qs[i] >> 4) & 0x0F0F0F0Fu), x.q[4 + i], s); // elements 16+4i..
    }
    return s - 8 * x.sumq;
}

// IQ3_S sub-block: qs0/qs1 its 8 index bytes, qh its high-bit byte, sg its 4
// sign bytes, nib its 4-bit scale; grid = codebook (LDS)
// Signed grid levels of an IQ3_S sub-block: word k (elements 4k..4k+3) is
// grid[qs[k] | (bit k of qh) << 8] with the bytes whose sign bit (bit 4k+i of
// sg) is set negated.  Indices are formed two at a time: v_perm interleaves
// two qs bytes with their high bits (bit k of qh spread to byte k) into two
// 16-bit indices, and one shift turns both into byte offsets of the table.
// Negation per byte: (g ^ m) + (m & 1) with m = 0xFF bytes, no carry across
// bytes since every level is >= 1.
// SG: grid is the sign-folded codebook (Iq3sSignedGrid in LDS)
template <bool SG = false>
__device__ __forceinline__ void iq3s_levels(uint32_t qs0, uint32_t qs1, uint32_t qh, uint32_t sg,
                                            const uint32_t* grid, uint32_t (&v)[8]) {
    const uint32_t h0 = nib_bits(qh & 0xFu), h1 = nib_bits((qh >> 4) & 0xFu);
    if constexpr (SG) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t pr = __builtin_amdgcn_perm(p < 2 ? h0 : h1, p < 2 ? qs0 : qs1,
                                                      (p & 1) ? 0x07030602u : 0x05010400u);
            // sign byte p: low nibble for word 2p, high nibble for word 2p+1,
            // placed as 4 * nibble in each 16-bit half beside 64 * index
            const uint32_t t = __mul24((sg >> (8 * p)) & 0xFFu, 0x4004u) & 0x003C003Cu;
            const uint32_t ab = (pr << 6) | t;
            v[2 * p] = *(const uint32_t*)((const uint8_t*)grid + (ab & 0xFFFFu));
            v[2 * p + 1] = *(const uint32_t*)((const uint8_t*)grid + (ab >> 16));
        }
        return;
    }
    uint32_t g[8];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        // bytes: qs[2p], hi bit 2p, qs[2p+1], hi bit 2p+1 (selector 0..3: src1 bytes, 4..7: src0 bytes)
        const uint32_t pr = __builtin_amdgcn_perm(p < 2 ? h0 : h1, p < 2 ? qs0 : qs1,
                                                  (p & 1) ? 0x07030602u : 0x05010400u);
        const uint32_t ab = pr << 2;                      // both indices times 4
        g[2 * p] = *(const uint32_t*)((const uint8_t*)grid + (ab & 0x7FCu));
        g[2 * p + 1] = *(const uint32_t*)((const uint8_t*)grid + (ab >> 16));
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {   // sign byte j: words 2j (low nibble), 2j+1
        uint32_t m0, m1;
        byte_sign_masks(sg, j, m0, m1);
        v[2 * j] = (g[2 * j] ^ m0) + (m0 & 0x01010101u);
        v[2 * j + 1] = (g[2 * j + 1] ^ m1) + (m1 & 0x01010101u);
    }
}

__device__ __forceinline__ int dot_iq3_s_core(uint32_t dbits, uint32_t qs0, uint32_t qs1, uint32_t qh, uint32_t sg,
                                              uint32_t nib, const XBlk& x, const uint32_t* grid, float* dw) {
    *dw = h2f(dbits);
    uint32_t v[8];
    iq3s_levels(qs0, qs1, qh, sg, grid, v);
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) s = dot4((int)v[k], x.q[k], s);
    return __mul24(s, 1 + 2 * (int)nib);
}
__device__ __forceinline__ int dot_q8_0(const uint8_t* row, int off, const XBlk& x, float* dw) {
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = lds_u32(row, off + 2 + 4 * i);
    return dot_q8_0_core(lds_u16(row, off), q, x, dw);
}

__device__ __forceinline__ int dot_q4_0(const uint8_t* row, int off, const XBlk& x, float* dw) {
    uint32_t qs[4];
#pragma unroll
    for (int i = 0; i < 4; i++) qs[i] = lds_u32(row, off + 2 + 4 * i);
    return dot_q4_0_core(lds_u16(row, off), qs, x, dw);
}

__device__ __forceinline__ int dot_iq3_s(const uint8_t* row, int off, int ib, const XBlk& x,
                                         const uint32_t* grid, float* dw) {
    const uint32_t sc = row[off + 106 + (ib >> 1)];
    return dot_iq3_s_core(lds_u16(row, off), lds_u32(row, off + 2 + 8 * ib), lds_u32(row, off + 6 + 8 * ib),
                          row[off + 66 + ib], lds_u32(row, off + 74 + 4 * ib), (sc >> (4 * (ib & 1))) & 0xFu, x,
                          grid, dw);
}

// ---- a weight block decoded once to 32 int8 values (8 words, element order
// of the Q8_1 block), for reuse against several activation blocks.
// wdot<T> gives the same exact sumi as the dot_* functions above (integer
// sums are order-free).  Q4_0 values are the raw nibbles (0..15); the -8
// term is applied with the activation's sum.  IQ3_S: signed grid levels and
// the sub-block multiplier 1 + 2*scale.
// Q4_K / Q5_K: unsigned quants 0..15 / 0..31, mult = 6-bit sub-block scale,
// plus the min term (dm = f32(dmin), mmin = 6-bit sub-block min).  Q6_K:
// signed quants q-32, mult / mult2 = the int8 scales of elements 0..15 /
// 16..31.  MXFP4: signed E2M1 levels doubled (int8), dw = 2^(e-128).
struct WBlk {
    int v[8];
    float dw;
    int mult;
    float dm;
    int mmin;
    int mult2;
};

template <int T>
__device__ __forceinline__ int wdot(const WBlk& w, const XBlk& x) {
    if constexpr (T == T_Q6_K) {
        // w.v holds the unsigned 6-bit quants u (0..63, valid non-negative
        // int8): sum (u - 32) q_x = sum u q_x - 32 sum q_x per 16-element half
        int lo = 0, hi = 0, slo = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo = dot4(w.v[i], x.q[i], lo);
            hi = dot4(w.v[4 + i], x.q[4 + i], hi);
            slo = dot4(x.q[i], 0x01010101, slo);
        }
        lo -= 32 * slo;
        hi -= 32 * (x.sumq - slo);
        return __mul24(lo, w.mult) + __mul24(hi, w.mult2);   // |.| <= 2 * 16*32*127*128 < 2^24
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = dot4(w.v[i], x.q[i], s);
    if constexpr (T == T_Q4_0) return s - 8 * x.sumq;
    else if constexpr (T == T_IQ3_S || T == T_Q4_K || T == T_Q5_K) return __mul24(s, w.mult);   // < 2^23
    else return s;
}

// One block's update of a lane accumulator in the documented fp32 order:
// acc = fmaf(f32(d_w)*f32(d_x), (float)sumi, acc); the K-quants with a min
// (Q4_K, Q5_K) then add fmaf(-(f32(dmin)*f32(d_x)), (float)(m * sum q_x), acc).
template <int T>
__device__ __forceinline__ float wacc(const WBlk& w, const XBlk& x, float acc) {
    if constexpr (T == T_Q4_0S) {
        // ggml's Q4_0 block term d_w * (sumi * d_x - 8 * s_x) with unsigned
        // nibbles in sumi, contracted as nvcc's default would: the inner
        // expression one fma, the product with d_w fused into the sum.  The
        // s field rides in sumq's slot of the decoded activation block.
        const float inner = __builtin_fmaf((float)wdot<T>(w, x), x.d, -(8.0f * h2f((uint32_t)x.sumq)));
        return __builtin_fmaf(w.dw, inner, acc);
    }
    acc = __builtin_fmaf(w.dw * x.d, (float)wdot<T>(w, x), acc);
    if constexpr (T == T_Q4_K || T == T_Q5_K) acc = __builtin_fmaf(-(w.dm * x.d), (float)__mul24(w.mmin, x.sumq), acc);
    return acc;
}

// Q8_1 blocks need the sum of their quants for these weight types
template <int T>
constexpr bool needs_sumq() { return T == T_Q4_0 || T == T_Q4_K || T == T_Q5_K || T == T_Q6_K; }

__device__ __forceinline__ void wdec_q8_0_core(uint32_t dbits, const uint32_t (&q)[8], WBlk& w) {
    w.dw = h2f(dbits);
    w.mult = 1;
#pragma unroll
    for (int i = 0; i < 8; i++) w.v[i] = (int)q[i];
}

__device__ __forceinline__ void wdec_q4_0_core(uint32_t dbits, const uint32_t (&qs)[4], WBlk& w) {
    w.dw = h2f(dbits);
    w.mult = 1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        w.v[i] = (int)(qs[i] & 0x0F0F0F0Fu);
        w.v[4 + i] = (int)((qs[i] >> 4) & 0x0F0F0F0Fu);
    }
}

template <bool SG = false>
__device__ __forceinline__ void wdec_iq3_s_core(uint32_t dbits, uint32_t qs0, uint32_t qs1, uint32_t qh, uint32_t sg,
                                                uint32_t nib, const uint32_t* grid, WBlk& w) {
    w.dw = h2f(dbits);
    w.mult = 1 + 2 * (int)nib;
    uint32_t v[8];
    iq3s_levels<SG>(qs0, qs1, qh, sg, grid, v);
#pragma unroll
    for (int k = 0; k < 8; k++) w.v[k] = (int)v[k];
}

// 6-bit scale and min of sub-block j (0..7) from the 12 packed scale bytes
// (as three little-endian words s0, s1, s2) of a Q4_K / Q5_K superblock
// (gguf_loader.rs:1150-1163): j < 4: sc = b[j] & 63, m = b[j+4] & 63;
// j >= 4: sc = (b[j+4] & 15) | (b[j-4] >> 6) << 4, m = (b[j+4] >> 4) | (b[j] >> 6) << 4.
// Branch-free: j varies across the lanes of a wave (a lane's sub-block), so
// both forms are formed from the same shifted words and one is selected.
__device__ __forceinline__ void kq_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int& sc, int& m) {
    const int k = 8 * (j & 3);
    const uint32_t a0 = s0 >> k, a1 = s1 >> k, a2 = s2 >> k;
    const uint32_t sc_hi = (a2 & 15u) | ((a0 & 0xC0u) >> 2), m_hi = ((a2 >> 4) & 15u) | ((a1 & 0xC0u) >> 2);
    sc = (int)(j < 4 ? a0 & 63u : sc_hi);
    m = (int)(j < 4 ? a1 & 63u : m_hi);
}

// Q4_K superblock (144 B: f16 d, f16 dmin, scales[12], qs[128]) sub-block ib
// (gguf_loader.rs:1265-1330): elements 32*ib + l = nibble (ib & 1) of
// qs[32*(ib/2) + l].  `sb` is 4-byte aligned.
__device__ __forceinline__ void wdec_q4_k(const uint8_t* sb, int ib, WBlk& w) {
    const uint32_t* u = (const uint32_t*)sb;
    w.dw = h2f(u[0] & 0xFFFFu);
    w.dm = h2f(u[0] >> 16);
    kq_scale_min(u[1], u[2], u[3], ib, w.mult, w.mmin);
    const int sh = 4 * (ib & 1);
    const uint32_t* qs = u + 4 + 8 * (ib >> 1);
#pragma unroll
    for (int i = 0; i < 8; i++) w.v[i] = (int)((qs[i] >> sh) & 0x0F0F0F0Fu);
    w.mult2 = 0;
}

// Q5_K superblock (176 B: f16 d, f16 dmin, scales[12], qh[32], qs[128])
// sub-block ib (gguf_loader.rs:1165-1263): the Q4_K nibble plus bit ib of
// qh[l] as bit 4.  `sb` is 4-byte aligned.
__device__ __forceinline__ void wdec_q5_k(const uint8_t* sb, int ib, WBlk& w) {
    const uint32_t* u = (const uint32_t*)sb;
    w.dw = h2f(u[0] & 0xFFFFu);
    w.dm = h2f(u[0] >> 16);
    kq_scale_min(u[1], u[2], u[3], ib, w.mult, w.mmin);
    const int sh = 4 * (ib & 1);
    const uint32_t* qh = u + 4;
    const uint32_t* qs = u + 12 + 8 * (ib >> 1);
    // bit ib of each qh byte to bit 4 of the byte: a rotate right by ib - 4
    // (mod 32) moves bit 8k + ib to bit 8k + 4 without crossing the word
    const uint32_t rot = (uint32_t)(ib - 4) & 31u;
#pragma unroll
    for (int i = 0; i < 8; i++)
        w.v[i] = (int)(((qs[i] >> sh) & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(qh[i], qh[i], rot) & 0x10101010u));
    w.mult2 = 0;
}

// Q6_K superblock (210 B: ql[128], qh[64], int8 scales[16], f16 d) sub-block
// ib = 4*gi + jj (gguf_loader.rs:839-917): element l (0..31) =
// (nibble (jj >> 1) of ql[64*gi + 32*(jj & 1) + l]) | ((qh[32*gi + l] >> 2*jj) & 3) << 4,
// minus 32; scale scales[8*gi + 2*jj + l/16].  `row` is a 4-byte aligned
// buffer, off the superblock's byte offset in it (even).  w.v holds the
// unsigned 6-bit values; wdot<T_Q6_K> applies the minus 32.
__device__ __forceinline__ void wdec_q6_k(const uint8_t* row, int off, int ib, WBlk& w) {
    const int gi = ib >> 2, jj = ib & 3;
    const int lo_off = off + 64 * gi + 32 * (jj & 1), hi_off = off + 128 + 32 * gi;
    // both runs share off's 2-byte phase a: read aligned words; one funnel
    // shift per word both realigns it and selects the nibble (lo) or the
    // 2-bit field (hi): bits 8a + shift .. of the word pair.  The quants stay
    // unsigned (0..63); wdot subtracts 32 per element through the block's sums
    const uint32_t a8 = 8u * (uint32_t)(off & 3);
    const uint32_t ls = a8 + 4u * (uint32_t)(jj >> 1), hs = a8 + 2u * (uint32_t)jj;
    const uint32_t* lw = (const uint32_t*)(row + (lo_off & ~3));
    const uint32_t* hw = (const uint32_t*)(row + (hi_off & ~3));
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t lo = __builtin_amdgcn_alignbit(lw[i + 1], lw[i], ls) & 0x0F0F0F0Fu;
        const uint32_t hx = __builtin_amdgcn_alignbit(hw[i + 1], hw[i], hs);
        w.v[i] = (int)(lo | ((hx << 4) & 0x30303030u));
    }
    const uint32_t scw = lds_u16(row, off + 192 + 8 * gi + 2 * jj);
    w.mult = (int)(int8_t)(scw & 0xFFu);
    w.mult2 = (int)(int8_t)(scw >> 8);
    w.dw = h2f(lds_u16(row, off + 208));
    w.dm = 0.0f;
    w.mmin = 0;
}

// 2^(e-128) as a float from the E8M0 byte e (the "half" scale of MXFP4:
// the element levels below are the E2M1 values doubled).
__device__ __forceinline__ float e8m0_half(uint32_t e) {
    const uint32_t bits = e >= 2 ? (e - 1) << 23 : 0x00200000u << e;
    return __builtin_bit_cast(float, bits);
}

// MXFP4 block (17 B: E8M0 e, qs[16]; element j = low nibble of qs[j],
// element j+16 = high nibble).  Nibble n -> level {0,1,2,3,4,6,8,12}[n & 7],
// negated when n & 8.  `row` 4-byte aligned buffer, off the block's offset.
__device__ __forceinline__ uint32_t mxfp4_levels(uint32_t nibs) {   // 4 nibbles in byte lanes
    const uint32_t sel = nibs & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
    const uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((nibs >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
    return (pos & ~m) | (neg & m);
}
__device__ __forceinline__ void wdec_mxfp4(const uint8_t* row, int off, WBlk& w) {
    w.dw = e8m0_half(row[off]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t q = lds_u32(row, off + 1 + 4 * i);
        w.v[i] = (int)mxfp4_levels(q & 0x0F0F0F0Fu);
        w.v[4 + i] = (int)mxfp4_levels((q >> 4) & 0x0F0F0F0Fu);
    }
    w.mult = 1;
    w.mult2 = 0;
    w.dm = 0.0f;
    w.mmin = 0;
}

// Block b of a row chunk in LDS (layout as block_dot below), decoded.  SG:
// IQ3_S lookups in the sign-folded codebook (Iq3sSignedGrid) instead of the
// 512-word one.
template <int T, bool SG = false>
__device__ __forceinline__ void block_decode(const uint8_t* row, int b, const uint32_t* grid, WBlk& w) {
    if constexpr (T == T_Q8_0) {
        const int off = b * 34;
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = lds_u32(row, off + 2 + 4 * i);
        wdec_q8_0_core(lds_u16(row, off), q, w);
    } else if constexpr (T == T_Q4_0 || T == T_Q4_0S) {
        const int off = b * 18;
        uint32_t qs[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = lds_u32(row, off + 2 + 4 * i);
        wdec_q4_0_core(lds_u16(row, off), qs, w);
    } else if constexpr (T == T_Q4_K) {
        wdec_q4_k(row + (b >> 3) * 144, b & 7, w);
    } else if constexpr (T == T_Q5_K) {
        wdec_q5_k(row + (b >> 3) * 176, b & 7, w);
    } else if constexpr (T == T_Q6_K) {
        wdec_q6_k(row, (b >> 3) * 210, b & 7, w);
    } else if constexpr (T == T_MXFP4) {
        wdec_mxfp4(row, b * 17, w);
    } else {
        const int off = (b >> 3) * 110, ib = b & 7;
        const uint32_t sc = row[off + 106 + (ib >> 1)];
        wdec_iq3_s_core<SG>(lds_u16(row, off), lds_u32(row, off + 2 + 8 * ib), lds_u32(row, off + 6 + 8 * ib),
                        row[off + 66 + ib], lds_u32(row, off + 74 + 4 * ib), (sc >> (4 * (ib & 1))) & 0xFu, grid, w);
    }
}

// One weight block held in registers, read straight from global memory with
// loads that never leave the block.  load() only issues the loads (the raw
// words are kept as loaded, so no wait is forced there); dot() assembles the
// fields on use.
template <int T> struct RegBlk;
template <> struct RegBlk<T_Q4_0> {
    // 18-byte block at an even address: 16-byte + 2-byte loads, ordered by the
    // block's 4-byte phase (ph = 0: [0,16) + [16,18); ph = 2: [0,2) + [2,18))
    static constexpr int LOADS = 2;   // vector-memory instructions issued by load()
    uint4 v;
    uint32_t t;
    bool ph2;
    __device__ __forceinline__ void load(const uint8_t* blk) {
        // no branch: the two loads of either phase are issued unconditionally
        ph2 = ((uintptr_t)blk & 3) != 0;
        v = *(const uint4*)(blk + (ph2 ? 2 : 0));
        t = *(const uint16_t*)(blk + (ph2 ? 0 : 16));
    }
    __device__ __forceinline__ void fields(uint32_t& d, uint32_t (&qs)[4]) const {
        if (!ph2) {
            d = v.x & 0xFFFFu;
            qs[0] = (v.x >> 16) | (v.y << 16);
            qs[1] = (v.y >> 16) | (v.z << 16);
            qs[2] = (v.z >> 16) | (v.w << 16);
            qs[3] = (v.w >> 16) | (t << 16);
        } else {
            d = t;
            qs[0] = v.x; qs[1] = v.y; qs[2] = v.z; qs[3] = v.w;
        }
    }
    __device__ __forceinline__ int dot(const XBlk& x, const uint32_t*, float* dw) const {
        uint32_t d, qs[4];
        fields(d, qs);
        return dot_q4_0_core(d, qs, x, dw);
    }
    __device__ __forceinline__ void decode(const uint32_t*, WBlk& w) const {
        uint32_t d, qs[4];
        fields(d, qs);
        wdec_q4_0_core(d, qs, w);
    }
};
template <> struct RegBlk<T_Q8_0> {
    // 34-byte block at an even address: two 16-byte loads and one 2-byte load
    static constexpr int LOADS = 3;
    uint4 v0, v1;
    uint32_t t;
    bool ph2;
    __device__ __forceinline__ void load(const uint8_t* blk) {
        ph2 = ((uintptr_t)blk & 3) != 0;
        const uint8_t* q = blk + (ph2 ? 2 : 0);
        v0 = *(const uint4*)q;
        v1 = *(const uint4*)(q + 16);
        t = *(const uint16_t*)(blk + (ph2 ? 0 : 32));
    }
    __device__ __forceinline__ int dot(const XBlk& x, const uint32_t*, float* dw) const {
        uint32_t d, q[8];
        fields(d, q);
        return dot_q8_0_core(d, q, x, dw);
    }
    __device__ __forceinline__ void decode(const uint32_t*, WBlk& w) const {
        uint32_t d, q[8];
        fields(d, q);
        wdec_q8_0_core(d, q, w);
    }
    __device__ __forceinline__ void fields(uint32_t& d, uint32_t (&q)[8]) const {
        if (!ph2) {
            const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, t};
            d = w[0] & 0xFFFFu;
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = (w[i] >> 16) | (w[i + 1] << 16);
        } else {
            d = t;
            q[0] = v0.x; q[1] = v0.y; q[2] = v0.z; q[3] = v0.w;
            q[4] = v1.x; q[5] = v1.y; q[6] = v1.z; q[7] = v1.w;
        }
    }
};
template <> struct RegBlk<T_IQ3_S> {
    // sub-block ib of a 110-byte superblock: its fields by 2-byte / 1-byte loads
    uint32_t d, q0, q1, q2, q3, qh, s0, s1, sc;
    int ib;
    __device__ __forceinline__ void load(const uint8_t* sb, int ib_) {
        ib = ib_;
        const uint16_t* h = (const uint16_t*)sb;
        d = h[0];
        q0 = h[1 + 4 * ib]; q1 = h[2 + 4 * ib]; q2 = h[3 + 4 * ib]; q3 = h[4 + 4 * ib];
        qh = sb[66 + ib];
        s0 = h[37 + 2 * ib]; s1 = h[38 + 2 * ib];
        sc = sb[106 + (ib >> 1)];
    }
    __device__ __forceinline__ int dot(const XBlk& x, const uint32_t* grid, float* dw) const {
        return dot_iq3_s_core(d, q0 | (q1 << 16), q2 | (q3 << 16), qh, s0 | (s1 << 16), (sc >> (4 * (ib & 1))) & 0xFu,
                              x, grid, dw);
    }
    __device__ __forceinline__ void decode(const uint32_t* grid, WBlk& w) const {
        wdec_iq3_s_core(d, q0 | (q1 << 16), q2 | (q3 << 16), qh, s0 | (s1 << 16), (sc >> (4 * (ib & 1))) & 0xFu, grid,
                        w);
    }
};

// Block b (32-element unit; IQ3_S: sub-block) of a row chunk held in LDS.
template <int T>
__device__ __forceinline__ int block_dot(const uint8_t* row, int b, const XBlk& x,
                                         const uint32_t* grid, float* dw) {
    if constexpr (T == T_Q8_0) return dot_q8_0(row, b * 34, x, dw);
    else if constexpr (T == T_Q4_0) return dot_q4_0(row, b * 18, x, dw);
    else return dot_iq3_s(row, (b >> 3) * 110, b & 7, x, grid, dw);
}

// cache policy of global->LDS weight copies: non-temporal (each weight byte is
// read once per call)
constexpr int CPOL_STREAM = 2;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// Copy `nrows` row segments of `seg` bytes (global row stride `gstride`) into
// LDS, packed with row stride `seg`.  When every piece is 16-byte (with DW:
// 4-byte) aligned the copy uses the asynchronous global->LDS loads
// (global_load_lds_dwordx4 / _dword: lane l of a wave deposits its 16 (4)
// bytes at a wave-uniform LDS base + 16*l (4*l)), so all loads of a phase are
// in flight together; otherwise all pieces are loaded to registers before any
// is stored.  The caller completes the copy with
// lds_copy_wait() + __syncthreads().
// stage_rows for a compile-time geometry: rows [0, n1) from g1 and [n1,
// nrows) from g2 (global row stride gstride), SEG-byte segments in UNIT-byte
// pieces (16: global_load_lds_dwordx4, 4: _dword; every piece UNIT-aligned),
// LDS row stride LSEG >= SEG (the padding is skipped), at most NRMAX rows, NTH
// threads.  Piece -> (row, column) by constant divisors and the loop fully
// unrolled, so a wave issues its copies back to back.  ONE: every row is g1's
// (n1 == nrows): each copy is the uniform base plus a 32-bit lane offset.
template <int SEG, int LSEG, int UNIT, int NRMAX, int NTH, int CPOL, bool ONE = false>
__device__ __forceinline__ void stage_rows_fixed(uint8_t* __restrict__ lds, const uint8_t* g1, int n1,
                                                 const uint8_t* g2, int64_t gstride, int nrows, int tid) {
    constexpr int PER = SEG / UNIT, LPER = LSEG / UNIT, NW = NTH / 64;
    constexpr int IT = (LPER * NRMAX + NTH - 1) / NTH;
    static_assert((UNIT == 16 || UNIT == 4) && SEG % UNIT == 0 && LSEG % UNIT == 0 && NTH % 64 == 0, "geometry");
    // lane through an empty asm: the piece addresses are formed here, next
    // to their copies, instead of being hoisted (registers) out of a caller's
    // chunk loop
    int lane = tid & 63;
    asm volatile("" : "+v"(lane));
    const int wave = tid >> 6;
    const unsigned tot = (unsigned)(LPER * nrows);
    // rows past n1 are g2's (32-bit offsets within a row run: gstride * rows < 2^31)
    const uintptr_t b2 = ONE ? 0 : (uintptr_t)g2 - (uintptr_t)((int64_t)n1 * gstride);
    const unsigned gs = (unsigned)gstride;
#pragma unroll
    for (int k = 0; k < IT; k++) {
        const int c0 = (k * NW + wave) * 64;
        const unsigned c = (unsigned)(c0 + lane);
        const unsigned r = c / LPER, col = c - r * LPER;
        if (c < tot && (LPER == PER || col < PER)) {
            const unsigned off = r * gs + col * UNIT;
            const uint8_t* src = ONE ? g1 + off : (const uint8_t*)(((int)r < n1 ? (uintptr_t)g1 : b2) + off);
            if constexpr (UNIT == 16)
                __builtin_amdgcn_global_load_lds((const glb_void_t*)src, (lds_void_t*)(lds + c0 * 16), 16, 0, CPOL);
            else
                __builtin_amdgcn_global_load_lds((const glb_void_t*)src, (lds_void_t*)(lds + c0 * 4), 4, 0, CPOL);
        }
    }
}

template <bool DW = false, int CPOL = 0>
__device__ __forceinline__ void stage_rows(uint8_t* __restrict__ lds, const uint8_t* __restrict__ g,
                                           int64_t gstride, int nrows, int seg, int tid, int nthreads,
                                           int lseg = 0) {
    // lseg: LDS row stride when it differs from seg (a padded stride, for the
    // 16-byte piece path only; the caller passes it only with seg % 16 == 0)
    if (lseg == 0) lseg = seg;
    const uintptr_t al = (uintptr_t)g | (uintptr_t)gstride | (uintptr_t)seg | (uintptr_t)lds;
    if (lseg != seg) {
        const int per = seg >> 4, lper = lseg >> 4, tot = lper * nrows;
        const int lane = tid & 63, wave = tid >> 6, nw = nthreads >> 6;
        for (int c0 = wave * 64; c0 < tot; c0 += nw * 64) {
            const int c = c0 + lane;
            const int r = c / lper, col = c - r * lper;
            if (c < tot && col < per)   // the rest of an LDS row is padding
                __builtin_amdgcn_global_load_lds((const glb_void_t*)(g + r * gstride + col * 16),
                                                 (lds_void_t*)(lds + c0 * 16), 16, 0, CPOL);
        }
    } else if (gstride == seg && (((uintptr_t)g | (uintptr_t)lds | (uintptr_t)(seg * nrows)) & 15) == 0) {
        // rows contiguous in memory and the whole run 16-byte aligned (even
        // when a row is not, e.g. 220-byte IQ3_S rows): one linear copy
        const int tot = seg * nrows / 16;
        const int lane = tid & 63, wave = tid >> 6, nw = nthreads >> 6;
        for (int c0 = wave * 64; c0 < tot; c0 += nw * 64) {
            const int c = c0 + lane;
            if (c < tot)
                __builtin_amdgcn_global_load_lds((const glb_void_t*)(g + c * 16), (lds_void_t*)(lds + c0 * 16), 16,
                                                 0, CPOL);
        }
    } else if ((al & 15) == 0) {
        const int per = seg >> 4, tot = per * nrows;
        const int lane = tid & 63, wave = tid >> 6, nw = nthreads >> 6;
        for (int c0 = wave * 64; c0 < tot; c0 += nw * 64) {
            const int c = c0 + lane;
            if (c < tot) {
                const int r = c / per, col = c - r * per;
                __builtin_amdgcn_global_load_lds((const glb_void_t*)(g + r * gstride + col * 16),
                                                 (lds_void_t*)(lds + c0 * 16), 16, 0, CPOL);
            }
        }
    } else if (DW && (al & 3) == 0) {
        // 4-byte aligned (e.g. IQ3_S chunks of 2 or 4 superblocks): the same
        // asynchronous copy in dword pieces (global_load_lds_dword)
        const int per = seg >> 2, tot = per * nrows;
        const int lane = tid & 63, wave = tid >> 6, nw = nthreads >> 6;
        for (int c0 = wave * 64; c0 < tot; c0 += nw * 64) {
            const int c = c0 + lane;
            if (c < tot) {
                const int r = c / per, col = c - r * per;
                __builtin_amdgcn_global_load_lds((const glb_void_t*)(g + r * gstride + col * 4),
                                                 (lds_void_t*)(lds + c0 * 4), 4, 0, CPOL);
            }
        }
    } else {
        // rare unaligned case: whole-dword or byte pieces, up to 8 in flight per thread
        const bool w4 = !DW && (al & 3) == 0;
        const int unit = w4 ? 4 : 1, per = seg / unit, tot = per * nrows;
        for (int i0 = 0; i0 < tot; i0 += 8 * nthreads) {
            uint32_t v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = i0 + k * nthreads + tid;
                if (i < tot) {
                    const int r = i / per, c = i - r * per;
                    v[k] = w4 ? *(const uint32_t*)(g + r * gstride + c * 4) : g[r * gstride + c];
                }
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = i0 + k * nthreads + tid;
                if (i < tot) {
                    if (w4) *(uint32_t*)(lds + i * 4) = v[k];
                    else lds[i] = (uint8_t)v[k];
                }
            }
        }
    }
}

// Asynchronous global->LDS copy, in one loop, of (1) n1 row segments of seg
// bytes at g1 + r*gstride and n2 at g2 + r*gstride, each as the 16-byte
// aligned span holding it (one piece per 16 bytes), to LDS rows of stride
// rs = 16 * pieces-per-row from `lds`, and (2) nx 16-byte pieces xsrc(i) to
// xlds + 16*i, starting at a multiple of 64 pieces so that each wave's 64
// lanes write one contiguous LDS run (the LDS address of these copies is
// wave-uniform).  One loop, because the compiler separates copy loops it
// cannot prove disjoint by a full wait.  Needs gstride % 16 == 0 and g1, g2
// at the same offset modulo 16 (every row then starts `pre` bytes into its
// LDS row: the return value; rs is returned in *rs_out).  Reads at most 15
// bytes beyond each end of a segment, inside the 16-byte granules holding
// its ends (so never outside a mapped page).
template <int CPOL, class XSrc>
__device__ __forceinline__ int stage_spans(uint8_t* __restrict__ lds, const uint8_t* g1, int n1, const uint8_t* g2,
                                           int n2, int64_t gstride, int seg, int* rs_out,
                                           uint8_t* __restrict__ xlds, int nx, XSrc xsrc, int tid, int nthreads,
                                           int minper = 0) {
    const int pre = (int)((uintptr_t)g1 & 15);
    const int per0 = (pre + seg + 15) >> 4, per = per0 > minper ? per0 : minper;   // copied pieces / LDS slots per row
    *rs_out = per * 16;
    const uint8_t* b1 = g1 - pre;
    const uint8_t* b2 = g2 - pre;
    const int t1 = per * n1, tw = t1 + per * n2;
    const int twp = (tw + 63) & ~63, tot = twp + nx;
    const int lane = tid & 63, wave = tid >> 6, nw = nthreads >> 6;
    for (int c0 = wave * 64; c0 < tot; c0 += nw * 64) {
        const int c = c0 + lane;
        if (c0 < twp) {
            if (c < tw) {
                const bool second = c >= t1;
                const int cc = second ? c - t1 : c;
                const int r = cc / per, col = cc - r * per;
                const uint8_t* src = (second ? b2 : b1) + r * gstride + col * 16;
                if (col < per0)
                    __builtin_amdgcn_global_load_lds((const glb_void_t*)src, (lds_void_t*)(lds + c0 * 16), 16, 0, CPOL);
            }
        } else if (c < tot) {
            __builtin_amdgcn_global_load_lds((const glb_void_t*)xsrc(c - twp), (lds_void_t*)(xlds + (c0 - twp) * 16),
                                             16, 0, 0);
        }
    }
    return pre;
}

// Waits for this thread's outstanding memory operations, including the
// asynchronous global->LDS copies; follow with __syncthreads().
__device__ __forceinline__ void lds_copy_wait() { __builtin_amdgcn_s_waitcnt(0); }

// s_waitcnt with only the vector-memory count: at most n outstanding
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// wait_vm with a run-time count n (0 <= n <= 15; larger n waits for 15)
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<1>(); break;
        case 2: wait_vm<2>(); break;
        case 3: wait_vm<3>(); break;
        case 4: wait_vm<4>(); break;
        case 5: wait_vm<5>(); break;
        case 6: wait_vm<6>(); break;
        case 7: wait_vm<7>(); break;
        case 8: wait_vm<8>(); break;
        case 9: wait_vm<9>(); break;
        case 10: wait_vm<10>(); break;
        case 11: wait_vm<11>(); break;
        case 12: wait_vm<12>(); break;
        case 13: wait_vm<13>(); break;
        case 14: wait_vm<14>(); break;
        default: wait_vm<15>(); break;
    }
}

// One 16-byte asynchronous global->LDS copy per lane (lane i writes
// lds_wave + 16 i; lds_wave must be the same for the whole wave).  Issued as
// inline assembly so that the compiler does not track it: it then inserts no
// vmcnt waits of its own before LDS reads it cannot prove disjoint from the
// copy, and the caller owns the wait (wait_vm, counted per wave in issue
// order) before reading the destination.  Compiler-tracked loads stay
// correct: an untracked copy issued after one of them only makes a vmcnt
// wait for it stricter.
__device__ __forceinline__ void copy16_lds_untracked(const void* g, void* lds_wave) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_wave);
    uint32_t saved;   // m0 is restored: compiler-generated code may keep a value there
    __asm__ volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
                     "s_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "v"(g), "s"(m)
                     : "memory");
}

// The dword form: lane l deposits its 4 bytes at lds_wave + 4*l
__device__ __forceinline__ void copy4_lds_untracked(const void* g, void* lds_wave) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_wave);
    uint32_t saved;
    __asm__ volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\t"
                     "s_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "v"(g), "s"(m)
                     : "memory");
}

// Work-group barrier that waits only for this wave's LDS accesses: the
// release fence of __syncthreads() would also wait for every outstanding
// asynchronous copy (they write LDS), including the next chunk's.  The empty
// asm statements keep memory accesses on their side of the barrier.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// Value of lane (lane ^ M) without going through LDS: DPP quad permutes for
// M = 1, 2, a half-row mirror plus a quad reversal for M = 4, a row rotation
// by 8 for M = 8, and the gfx950 v_permlane16/32_swap for M = 16, 32.  The partner lane must be
// active (all uses keep whole 2M-lane groups converged).
template <int M>
__device__ __forceinline__ int xlane(int v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "xor mask");
    const int lane = __lane_id();
    if constexpr (M == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    else if constexpr (M == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); // quad_perm 2,3,0,1
    else if constexpr (M == 4) {
        // row_half_mirror (i -> 7-i in each 8-lane half) then quad_perm 3,2,1,0:
        // lane i ends with lane (i & ~7) | (7 - ((i & 4) | (3 - (i & 3)))) = i ^ 4
        const int hm = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
        return __builtin_amdgcn_update_dpp(0, hm, 0x1B, 0xF, 0xF, false);
    } else if constexpr (M == 8) {
        return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);   // row_ror:8 = xor 8 in a 16-lane row
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((lane & 16) ? r[0] : r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((lane & 32) ? r[0] : r[1]);
    }
}
template <int M>
__device__ __forceinline__ float xlane(float v) {
    return __builtin_bit_cast(float, xlane<M>(__builtin_bit_cast(int, v)));
}

// Maximum of a non-negative int over the wave, returned wave-uniform: DPP
// prefix maximum (row_shr 1, 2, 4, 8 inside each 16-lane row, then
// row_bcast 15 / 31 across rows) leaves the total in lane 63.
__device__ __forceinline__ int wave_max_nonneg(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false));   // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false));   // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false));   // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false));   // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false));   // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false));   // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// Inclusive prefix sum of a non-negative int over the wave (Hillis-Steele:
// row_shr 1, 2, 4, 8 inside each 16-lane row, then row_bcast 15 / 31 carry
// the row totals forward).
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);   // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);   // row_bcast:31
    return v;
}

// Sum over the 16 lanes of a row group in the halving-tree order
// (xor 8, 4, 2, 1); every lane of the group ends with the same value.
__device__ __forceinline__ float slot_reduce16(float v) {
    v = v + xlane<8>(v);
    v = v + xlane<4>(v);
    v = v + xlane<2>(v);
    v = v + xlane<1>(v);
    return v;
}

// 32-lane xor butterflies (masks 16, 8, 4, 2, 1): max and sum
__device__ __forceinline__ float bfly32_max(float v) {
    v = __builtin_fmaxf(v, xlane<16>(v));
    v = __builtin_fmaxf(v, xlane<8>(v));
    v = __builtin_fmaxf(v, xlane<4>(v));
    v = __builtin_fmaxf(v, xlane<2>(v));
    return __builtin_fmaxf(v, xlane<1>(v));
}
__device__ __forceinline__ float bfly32_sum(float v) {
    v = v + xlane<16>(v);
    v = v + xlane<8>(v);
    v = v + xlane<4>(v);
    v = v + xlane<2>(v);
    return v + xlane<1>(v);
}

}  // namespace chimere
