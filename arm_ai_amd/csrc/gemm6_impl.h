// gemm6_impl.h -- the f16-MFMA prefill GEMM for Q6_K and Q5_K weights: its
// types, kernel body and launch plan, shared by k_gemm6.hip (its own
// launches) and k_gemm.hip (a launch that runs it beside the Q4_K GEMM).  The
// method is described at the top of k_gemm6.hip.
#pragma once

#include "aq_internal.h"

#include <algorithm>
#include <type_traits>

namespace aq {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int G6N = 128;  // columns (n) per workgroup
constexpr int G6M = 64;   // rows (m) per workgroup
constexpr int NXCD6 = 8;
constexpr int TARGET_WG6 = 512;  // two workgroups per CU

struct Gemm6Params {
    const uint8_t *w;     // row-block tiles
    const uint16_t *wd;   // d plane [n/8][ng][8] f16
    int64_t rb_stride;
    int ng;
    const uint16_t *x16;  // activation quants as f16 [m][k]
    const float *xd;      // [m][ng]
    const uint16_t *xbs;  // Q5_K: bsums as f16 [m][k/16]
    float *y;
    int m, n, k;
    int ntm, tiles, splits, kbs, items, per_xcd;
    float *part;          // [tiles][splits][64][128] (splits > 1)
    int32_t *S, *Smin;    // integer dump [m][n][ng] or null (Q6_K has no min term: Smin zeros)
};

// One lane's weight bytes of one super-block: bytes 8h..8h+7 of the 8 ql and
// 4 qh pieces of its column, the 16 int8 scales, and d.
struct W6 {
    u32x2 ql[8], qh[4];
    u32x4 sc;
    uint32_t d;
};

// One lane's weight bytes of one Q5_K super-block: bytes 8h..8h+7 of the 8 qs
// and 2 qh pieces of its column, and the whole of piece 0 (d, dmin, scales).
struct W5 {
    u32x2 qs[8], qh[2];
    u32x4 meta;
};

struct Lds6 {
    static constexpr int QS = G6M * 512;  // f16 quants [64 rows][256], chunk c of row r at c ^ (r & 31)
    static constexpr int DX = QS;         // d_x [64] f32
    static constexpr int BS = QS + 256;   // Q5_K: bsums [64 rows][16] f16
    static constexpr int STAGE = BS + G6M * 32;
    static constexpr int BYTES = 2 * STAGE;
};

__device__ __forceinline__ void load_w6(W6 &W, const rsrc_t &rw, const rsrc_t &rwd, uint32_t off, uint32_t doff,
                                        int b, int ng) {
    const bool ok = b < ng;
    const uint32_t o = ok ? off + (uint32_t)(b * 13 * 128) : BUF_OOB;
#pragma unroll
    for (int i = 0; i < 8; i++) W.ql[i] = __builtin_amdgcn_raw_buffer_load_b64(rw, o + i * 128, 0, BUF_NT);
#pragma unroll
    for (int i = 0; i < 4; i++) W.qh[i] = __builtin_amdgcn_raw_buffer_load_b64(rw, o + (8 + i) * 128, 0, BUF_NT);
    // the scales piece: the whole 16 bytes (this lane's h offset removed)
    W.sc = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (o & ~15u) + 12 * 128 : BUF_OOB, 0, BUF_NT);
    W.d = __builtin_amdgcn_raw_buffer_load_b16(rwd, ok ? doff + (uint32_t)(b * RB * 2) : BUF_OOB, 0, BUF_NT);
}

// The 8 f16 weight operands of sub-block j for this lane (elements 16j + 8h
// .. 16j + 8h + 7 of its column's super-block), for the two digits of the
// sub-scale: rh = sh * (q6 - 32), rl = sl * (q6 - 32), sc_j = 16 sh + sl.
__device__ __forceinline__ void w6_operands(const W6 &W, int j, v8h &rh, v8h &rl) {
    const int hh = j >> 3, jj = j & 7, qq = jj >> 1, odd = jj & 1;
    const u32x2 ql = W.ql[4 * hh + 2 * (qq & 1) + odd];
    const u32x2 qh = W.qh[2 * hh + odd];
    uint32_t q[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t nib = (qq >> 1) ? (ql[i] >> 4) & 0x0F0F0F0Fu : ql[i] & 0x0F0F0F0Fu;
        const uint32_t hb = (qq < 2 ? qh[i] << (4 - 2 * qq) : qh[i] >> (2 * qq - 4)) & 0x30303030u;
        q[i] = nib | hb;
    }
    const int sc = (int)(int8_t)((W.sc[j >> 2] >> (8 * (j & 3))) & 0xffu);
    const int sh = sc >> 4, sl = sc & 15;  // arithmetic shift: sc = 16 * sh + sl
    const _Float16 fh = (_Float16)sh, oh = (_Float16)(-1056 * sh);  // |1056 sh| <= 2^8 * 33: exact
    const _Float16 fl = (_Float16)sl, ol = (_Float16)(-1056 * sl);  // 1056 sl <= 2^5 * 495: exact
    const h2 sh2 = {fh, fh}, oh2 = {oh, oh}, sl2 = {fl, fl}, ol2 = {ol, ol};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // bytes 2i, 2i+1 of q as 16-bit lanes, then 1024 + q as f16
        const uint32_t u = __builtin_amdgcn_perm(0u, q[i >> 1], (i & 1) ? 0x0C030C02u : 0x0C010C00u) | 0x64006400u;
        const h2 f = __builtin_bit_cast(h2, u);
        const h2 vh = __builtin_elementwise_fma(f, sh2, oh2);
        const h2 vl = __builtin_elementwise_fma(f, sl2, ol2);
        rh[2 * i] = vh[0];
        rh[2 * i + 1] = vh[1];
        rl[2 * i] = vl[0];
        rl[2 * i + 1] = vl[1];
    }
}

__device__ __forceinline__ void load_w5(W5 &W, const rsrc_t &rw, uint32_t off, int b, int ng) {
    const bool ok = b < ng;
    const uint32_t o = ok ? off + (uint32_t)(b * 11 * 128) : BUF_OOB;
    // piece 0 whole (this lane's h offset removed), then qh, then qs
    W.meta = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? o & ~15u : BUF_OOB, 0, BUF_NT);
#pragma unroll
    for (int i = 0; i < 2; i++) W.qh[i] = __builtin_amdgcn_raw_buffer_load_b64(rw, o + (1 + i) * 128, 0, BUF_NT);
#pragma unroll
    for (int i = 0; i < 8; i++) W.qs[i] = __builtin_amdgcn_raw_buffer_load_b64(rw, o + (3 + i) * 128, 0, BUF_NT);
}

// The 8 f16 weight operands sc * q5 of MFMA j, elements 16j + 8h .. 16j + 8h + 7
// of this lane's column's super-block: chunk c = j / 4 of 64 elements, low
// nibbles of qs[32c ..] for its first 32 elements and high nibbles for the
// rest, the fifth bit from qh bit 2c (low) or 2c + 1 (high); sub-block j / 2.
__device__ __forceinline__ v8h w5_operand(const W5 &W, int j, uint32_t sc) {
    const int c = j >> 2, hi = (j >> 1) & 1, odd = j & 1;
    const u32x2 qs = W.qs[2 * c + odd];
    const u32x2 qh = W.qh[odd];
    uint32_t q[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t nib = hi ? (qs[i] >> 4) & 0x0F0F0F0Fu : qs[i] & 0x0F0F0F0Fu;
        q[i] = nib | (((qh[i] >> (2 * c + hi)) & 0x01010101u) << 4);
    }
    const _Float16 s = (_Float16)(int)sc;
    const _Float16 o = (_Float16)(-1024 * (int)sc);  // exact: sc * 2^10 <= 64512
    const h2 s2 = {s, s}, o2 = {o, o};
    v8h r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t u = __builtin_amdgcn_perm(0u, q[i >> 1], (i & 1) ? 0x0C030C02u : 0x0C010C00u) | 0x64006400u;
        const h2 f = __builtin_bit_cast(h2, u);
        const h2 v = __builtin_elementwise_fma(f, s2, o2);
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

// The kernel's body for workgroup bid of the launch, on LDS of Lds6::BYTES
// (so that another launch can run it beside other work).
template <int TYPE, bool DUMP>
__device__ __forceinline__ void gemm_f16w_body(Gemm6Params p, uint8_t *lds, int bid) {
    constexpr bool Q5 = TYPE == TYPE_Q5_K;
    const int xcd = bid % NXCD6, local = bid / NXCD6;
    const int item = xcd * p.per_xcd + local;
    if (local >= p.per_xcd || item >= p.items) return;  // uniform over the workgroup
    const int tile = item / p.splits, split = item - tile * p.splits;
    const int tn = tile / p.ntm, tm = tile - tn * p.ntm;
    const int m0 = tm * G6M;
    const int kb0 = split * p.kbs;
    const int kb1 = min(p.ng, kb0 + p.kbs);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    const int ccol = wave * 32 + l32;
    const int col = tn * G6N + ccol;
    const bool col_ok = col < p.n;
    const int ng = p.ng, k = p.k;

    // activation copies: instruction i of wave w fills LDS bytes (8w+i)*1024 +
    // 16*lane: row r = 2(8w+i) + lane/32, chunk position lane%32, which holds
    // the row's chunk (lane%32) ^ (r & 31).  Rows past m read zeros.
    const rsrc_t rq = buf_rsrc(p.x16, (uint32_t)((int64_t)p.m * k * 2));
    const rsrc_t rdx = buf_rsrc(p.xd, (uint32_t)((int64_t)p.m * ng * 4));
    uint32_t qoff[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = 2 * (8 * wave + i) + (lane >> 5), cp = lane & 31;
        qoff[i] = (uint32_t)((m0 + r) * k * 2 + 16 * (cp ^ (r & 31)));
    }
    const uint32_t dxoff = (uint32_t)((m0 + lane) * ng * 4);
    // Q5_K bsums: waves 1 and 2 copy rows 0..31 and 32..63, lane L row L / 2,
    // groups 8 (L % 2) .. 8 (L % 2) + 7
    const rsrc_t rbs = buf_rsrc(p.xbs, Q5 ? (uint32_t)((int64_t)p.m * (k / 16) * 2) : 0u);
    const uint32_t bsoff = (uint32_t)(((m0 + 32 * ((wave - 1) & 1) + (lane >> 1)) * (k / 16) + 8 * (lane & 1)) * 2);
    // weights: this lane's column is row (ccol % 8) of the tile's row block ccol / 8
    const int nrb = (p.n + RB - 1) / RB;
    const int rb_here = min(16, nrb - 16 * tn);
    const rsrc_t rw = buf_rsrc(p.w + (int64_t)16 * tn * p.rb_stride, (uint32_t)(rb_here * p.rb_stride));
    const rsrc_t rwd = Q5 ? rw : buf_rsrc(p.wd + (int64_t)16 * tn * ng * RB, (uint32_t)(rb_here * ng * RB * 2));
    const uint32_t woff = (uint32_t)((ccol >> 3) * p.rb_stride + (ccol & 7) * 16 + 8 * h);
    const uint32_t wdoff = (uint32_t)((((ccol >> 3) * ng) * RB + (ccol & 7)) * 2);

    // b past the range (the step after the last) re-reads the last super-block:
    // the scalar offset is kept inside the buffers
    auto issue = [&](uint8_t *st, int b) {
        b = min(b, kb1 - 1);
#pragma unroll
        for (int i = 0; i < 8; i++) buf_to_lds16(rq, st + 1024 * (8 * wave + i), qoff[i], b * 512);
        if (wave == 0) buf_to_lds4(rdx, st + Lds6::DX, dxoff, b * 4);  // wave-uniform
        if (Q5 && (wave == 1 || wave == 2)) buf_to_lds16(rbs, st + Lds6::BS + 1024 * (wave - 1), bsoff, b * 32);
    };

    v16f yacc[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) yacc[t][r] = 0.0f;

    auto read_a = [&](const uint8_t *st, int t, int j) {
        const int R = 32 * t + l32, C = 2 * j + h;
        return *(const v8h *)(st + R * 512 + 16 * (C ^ (R & 31)));
    };

    auto compute6 = [&](const uint8_t *st, const W6 &W, int b) {
        v16f acc[2][2];  // [tile][high / low digit of the sub-scales]
#pragma unroll
        for (int j = 0; j < 16; j++) {
            v8h bh, bl;
            w6_operands(W, j, bh, bl);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const v16f z = {0};
                const v8h a = read_a(st, t, j);
                acc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, j == 0 ? z : acc[t][0], 0, 0, 0);
                acc[t][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, j == 0 ? z : acc[t][1], 0, 0, 0);
            }
        }
        const float dw = f16_bits_to_f32(W.d);
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const v4f dx4 = *(const v4f *)(st + Lds6::DX + 4 * (32 * t + 8 * g4 + 4 * h));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g4 + i;
                    // f32 combine: y += (d_w * d_x) * S, S = 16 A_h + A_l
                    yacc[t][r] = __builtin_fmaf(dw * dx4[i], __builtin_fmaf(16.0f, acc[t][0][r], acc[t][1][r]), yacc[t][r]);
                    if (DUMP) {
                        const int row = m0 + 32 * t + 8 * g4 + 4 * h + i;
                        if (row < p.m && col_ok) {
                            const int64_t o = ((int64_t)row * p.n + col) * ng + b;
                            p.S[o] = 16 * (int)acc[t][0][r] + (int)acc[t][1][r];
                            p.Smin[o] = 0;
                        }
                    }
                }
            }
        }
    };

    auto compute5 = [&](const uint8_t *st, const W5 &W, int b) {
        // scales / mins of this lane's column (candle's utmp form of get_scale_min_k4)
        const uint32_t u0 = W.meta.y, u1 = W.meta.z, u2 = W.meta.w;
        const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
        const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
        const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
        // chain c (sub-blocks 2c, 2c + 1) is exact; S in f32 = ((c0 + c1) + c2) + c3,
        // folded as each chain ends; the dump keeps the chains for the int32 sum
        v16f cur[2], tot[2], keep[2][DUMP ? 4 : 1];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int sb = j >> 1;
            const uint32_t sc = ((sb < 4 ? sc03 : sc47) >> (8 * (sb & 3))) & 0xffu;
            const v8h bw = w5_operand(W, j, sc);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const v16f z = {0};
                cur[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_a(st, t, j), bw, (j & 3) == 0 ? z : cur[t], 0, 0, 0);
                if ((j & 3) == 3) {
                    tot[t] = j == 3 ? cur[t] : tot[t] + cur[t];
                    if (DUMP) keep[t][DUMP ? j >> 2 : 0] = cur[t];
                }
            }
        }
        // Smin: A[m][g] = bsums (g = 8h + i), B[g][n] = mn[g/2]
        const uint32_t mw = h ? mn47 : mn03;
        v8h bmn;
#pragma unroll
        for (int i = 0; i < 8; i++) bmn[i] = (_Float16)(int)((mw >> (8 * (i >> 1))) & 0xffu);
        v16f sm[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const v8h abs = *(const v8h *)(st + Lds6::BS + (32 * t + l32) * 32 + 16 * h);
            const v16f z = {0};
            sm[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(abs, bmn, z, 0, 0, 0);
        }
        const float dw = f16_bits_to_f32(W.meta.x), dmw = f16_bits_to_f32(W.meta.x >> 16);
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const v4f dx4 = *(const v4f *)(st + Lds6::DX + 4 * (32 * t + 8 * g4 + 4 * h));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * g4 + i;
                    // f32 combine: y += d_x * (d_w * S - dmin_w * Smin)
                    yacc[t][r] = __builtin_fmaf(dx4[i], __builtin_fmaf(-dmw, sm[t][r], dw * tot[t][r]), yacc[t][r]);
                    if (DUMP) {
                        const int row = m0 + 32 * t + 8 * g4 + 4 * h + i;
                        if (row < p.m && col_ok) {
                            const int64_t o = ((int64_t)row * p.n + col) * ng + b;
                            int si = 0;
#pragma unroll
                            for (int c = 0; c < (DUMP ? 4 : 1); c++) si += (int)keep[t][c][r];
                            p.S[o] = si;
                            p.Smin[o] = (int)sm[t][r];
                        }
                    }
                }
            }
        }
    };

    using WR = typename std::conditional<Q5, W5, W6>::type;
    auto load_w = [&](WR &W, int b) {
        if constexpr (Q5) load_w5(W, rw, woff, b, kb1);
        else load_w6(W, rw, rwd, woff, wdoff, b, kb1);
    };
    auto compute = [&](const uint8_t *st, const WR &W, int b) {
        if constexpr (Q5) compute5(st, W, b);
        else compute6(st, W, b);
    };

    // Two main stages and two weight register sets, one super-block ahead:
    // step b waits for its copies and loads (all this wave's outstanding
    // memory operations), a barrier, then issues step b + 1's.
    WR wa, wb;
    issue(lds, kb0);
    load_w(wa, kb0);
    for (int b = kb0; b < kb1; b += 2) {
        wait_vmcnt<0>();
        stage_barrier();
        issue(lds + Lds6::STAGE, b + 1);
        load_w(wb, b + 1);  // past kb1: zeros
        compute(lds, wa, b);
        if (b + 1 >= kb1) break;
        wait_vmcnt<0>();
        stage_barrier();
        issue(lds, b + 2);
        load_w(wa, b + 2);
        compute(lds + Lds6::STAGE, wb, b + 1);
    }
    wait_vmcnt<0>();  // no copy may still be landing when the workgroup ends

    if (p.splits == 1) {
        if (col_ok) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < p.m) p.y[(int64_t)row * p.n + col] = yacc[t][r];
                }
        }
        return;
    }
    float *mine = p.part + ((int64_t)tile * p.splits + split) * (G6M * G6N);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) mine[(32 * t + 8 * (r >> 2) + 4 * h + (r & 3)) * G6N + ccol] = yacc[t][r];
}

template <int TYPE, bool DUMP>
__global__ __launch_bounds__(256, 2) void gemm_f16w_kernel(Gemm6Params p) {
    __shared__ __align__(16) uint8_t lds[Lds6::BYTES];
    gemm_f16w_body<TYPE, DUMP>(p, lds, (int)blockIdx.x);
}

// The activation quants as f16 (exact), four per thread.
__global__ __launch_bounds__(256) void qs_to_f16_kernel(const int8_t *__restrict__ qs, int64_t n4,
                                                        uint16_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const uint32_t q = ((const uint32_t *)qs)[i];
    uint16_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = __builtin_bit_cast(uint16_t, (_Float16)(int)(int8_t)((q >> (8 * j)) & 0xffu));
    ((uint2 *)out)[i] = make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
}

struct Gemm6Plan {
    int ntm, ntn, tiles, splits, kbs;
    size_t part, ws;
};

// 64 x 128 tiles, two workgroups per CU; K split while there are fewer items
// than workgroup slots, each split keeping at least two super-blocks.  (The
// kernel is latency-bound at one workgroup per CU: a split that leaves the
// same number of rounds still pays for itself, e.g. 352 tiles x 8
// super-blocks in 30 us with two splits plus a 10 us reduce, 44 us without.)
Gemm6Plan gemm6_plan(int64_t m, int64_t n, int64_t k) {
    Gemm6Plan g;
    const int ng = (int)(k / QK_K);
    g.ntn = (int)((n + G6N - 1) / G6N);
    g.ntm = (int)((m + G6M - 1) / G6M);
    g.tiles = g.ntm * g.ntn;
    g.splits = 1;
    while ((int64_t)g.tiles * g.splits < TARGET_WG6 && ng / (2 * g.splits) >= 2) g.splits *= 2;
    g.kbs = (ng + g.splits - 1) / g.splits;
    g.splits = (ng + g.kbs - 1) / g.kbs;
    g.part = g.splits > 1 ? (size_t)g.tiles * g.splits * G6M * G6N * 4 : 0;
    g.ws = align_up(g.part, 256) + align_up((size_t)m * k * 2, 256);  // partials, then the f16 activation
    return g;
}

int64_t gemm6_chunk_rows(int64_t k) {
    const int64_t cap = (((int64_t)1 << 31) - 1) / (2 * k) / 64 * 64;  // f16 activation offsets in 32 bits
    return cap;
}

}  // namespace

}  // namespace aq
