// k_gemm8.hip -- prefill GEMM (m > 8) for Q8_0 weights on the int8 matrix
// cores, gfx950.
//
// Replaces the M-row loop of candle-core 0.8.4 k_quants::matmul<BlockQ8_0>
// at prefill (native/arm_ai_nif/src/llama_candle.rs:93; the activation is
// quantised to Q8_0 blocks, BlockQ8_0::vec_dot per 32-element block):
//   y[m][n] = sum_b (f32)S_b * f16(d_w[n,b]) * f16(d_x[m,b]),
//   S_b = sum_{e in b} qw_e * qx_e  (exact in i32).
//
// One v_mfma_i32_32x32x32_i8 covers one block (K = 32) of a 32 x 32 tile.
// The per-block scaling is the whole cost beyond the MFMA, so it is cut to
// two f32 fmas per output:
//   - The MFMA does not start from zero but from the constant C0 = 0x4B400000,
//     the bits of 1.5 * 2^23.  Its i32 result C0 + S, read as f32, is exactly
//     1.5 * 2^23 + S (|S| <= 32 * 128 * 127 < 2^22 keeps the exponent fixed):
//     the int -> float conversion is free.
//   - t = fma(C0 + S, d_w, -1.5 * 2^23 * d_w) rounds S * d_w once, so it is
//     bit-identical to candle's (f32)S * d_w (the constant product is exact:
//     d_w has an 11-bit significand).
//   - acc = fma(t, d_x, acc): one rounding fewer than candle's mul-then-add
//     (within the f32 tolerance of the output; the integer sums are bit-exact,
//     see the dump variant).
//
// Tiling.  A workgroup (4 wavefronts, two workgroups per CU) owns a 128 (m) x
// 128 (n) tile; each wavefront a 64 x 64 block of four 32 x 32 MFMA tiles.
// A step is 64 k-bytes (two blocks).  Per step, buffer loads into LDS copy:
//   - the 128 activation rows' 64 quant bytes (16-byte chunks at position
//     c ^ ((r >> 2) & 3) of the row, so 16 consecutive rows read
//     conflict-free);
//   - the 16 row blocks' four 128-byte weight lines (pieces 4s..4s+3 of group
//     g = step / 4, s = step % 4), in their tile order [row block][piece][row];
//   - d_x of both blocks for the 128 rows, gathered 4 bytes per lane into
//     [block][row] order (four consecutive rows of a lane's MFMA output are
//     then one 16-byte read);
//   - the 128 columns' two f16 d_w (4 bytes of piece 16 of the group).
// Four stages, issued three steps ahead.  Work items (tile, k-split) are
// dealt so that all m-tiles and k-splits of one n-tile run on one XCD and
// share its L2 copy of the weight rows.  Split-K partial tiles are summed in
// split order by the Q4_K GEMM's reduce launch.
#include "aq_internal.h"

#include <algorithm>

namespace aq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int G8T = 128;     // rows (m) and columns (n) per workgroup tile
constexpr int G8K = 64;      // k-bytes per step: two Q8_0 blocks
constexpr int G8NST = 4;     // stages in the LDS ring
constexpr int G8XCD = 8;
constexpr int TARGET_WG8 = 512;  // two workgroups per CU
constexpr int G8COPIES = 6;      // copy instructions per wavefront and step
constexpr int32_t C0 = 0x4B400000;   // bits of 1.5 * 2^23
constexpr float C0F = 12582912.0f;   // 1.5 * 2^23

struct L8 {
    static constexpr int ACT = 0;                 // [128 rows][64 B], swizzled chunks
    static constexpr int W = G8T * G8K;           // [16 row blocks][4 pieces][8 rows][16 B]
    static constexpr int DX = 2 * G8T * G8K;      // [2 blocks][128 rows] f32
    static constexpr int DW = DX + 2 * G8T * 4;   // [128 columns] two f16
    static constexpr int PAD = DW + G8T * 4;      // landing area of the unused gather lanes
    static constexpr int STAGE = PAD + 2 * 256;
};
static_assert(L8::STAGE * G8NST * 2 <= 160 * 1024, "two workgroups per CU");

struct Gemm8Params {
    const uint8_t *w;      // row-block tiles
    int64_t rb_stride;
    int ng;                // groups (8 blocks) per weight row
    const int8_t *xq;      // [m][k] quants
    const float *xd;       // [m][k/32] d_x
    float *y;              // [m][n]
    float *part;           // split-K partial tiles
    int32_t *S, *Smin;     // integer dump [m][n][k/32] (DUMP only)
    int m, n, k, nb;       // nb = k / 32
    int ntm, tiles, splits, kss, items, per_xcd;  // kss: steps per split
};

template <bool DUMP>
__global__ __launch_bounds__(256, 2) void gemm_q80_kernel(const Gemm8Params p) {
    __shared__ __align__(16) uint8_t lds[G8NST * L8::STAGE];
    const int xcd = blockIdx.x % G8XCD, local = blockIdx.x / G8XCD;
    const int item = xcd * p.per_xcd + local;
    if (local >= p.per_xcd || item >= p.items) return;  // uniform over the workgroup
    const int tile = item / p.splits, split = item - tile * p.splits;
    const int tn = tile / p.ntm, tm = tile - tn * p.ntm;
    const int m0 = tm * G8T, n0 = tn * G8T;
    const int nk = (p.nb + 1) / 2;  // steps over the whole row
    const int ks0 = split * p.kss, ks1 = min(nk, ks0 + p.kss);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, l32 = lane & 31;
    const int k = p.k;

    const rsrc_t ra = buf_rsrc(p.xq, (uint32_t)((int64_t)p.m * k));
    const rsrc_t rdx = buf_rsrc(p.xd, (uint32_t)((int64_t)p.m * p.nb * 4));
    const int rb0 = n0 / 8, rb_all = (p.n + 7) / 8;
    const int rb_here = min(G8T / 8, rb_all - rb0);
    const rsrc_t rw = buf_rsrc(p.w + (int64_t)rb0 * p.rb_stride, (uint32_t)(rb_here * p.rb_stride));

    // Per-lane offsets (fixed over the steps; the step enters as the scalar
    // offset).  Copy instruction i of this wavefront, q = 2 * wave + i:
    //   activations: LDS chunk t = 64q + lane -> row t/4, position t%4,
    //                holding the row's chunk (t%4) ^ ((row >> 2) & 3);
    //   weights:     row blocks 2q, 2q+1; lane -> (row block 2q + lane/32,
    //                piece (lane%32)/8, row lane%8), 16 bytes;
    //   gathers:     q 0..3 -> d_x of block q/2, rows 64(q%2) + lane;
    //                q 4, 5 -> d_w pair of columns 64(q-4) + lane;
    //                q 6, 7 -> unused (read out of range into the pad).
    uint32_t aoff[2], woff[2], goff[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int q = 2 * wave + i;
        const int t = 64 * q + lane, r = t >> 2, cp = t & 3;
        const int64_t ao = (int64_t)(m0 + r) * k + 16 * (cp ^ ((r >> 2) & 3));
        aoff[i] = m0 + r < p.m ? (uint32_t)ao : BUF_OOB;  // rows past m read zeros
        woff[i] = (uint32_t)((int64_t)(2 * q + (lane >> 5)) * p.rb_stride + (lane & 31) * 16);
        if (q < 4) {
            const int row = m0 + 64 * (q & 1) + lane;
            goff[i] = (uint32_t)(((int64_t)row * p.nb + (q >> 1)) * 4);
        } else if (q < 6) {
            const int c = 64 * (q - 4) + lane;
            goff[i] = (uint32_t)((int64_t)(c >> 3) * p.rb_stride + 16 * 128 + (c & 7) * 16);
        } else {
            goff[i] = BUF_OOB;
        }
    }
    uint8_t *const gdst0 = lds + (2 * wave < 4 ? L8::DX + 256 * (2 * wave) : 2 * wave < 6 ? L8::DW + 256 * (2 * wave - 4)
                                                                                          : L8::PAD);
    auto issue = [&](int slot_ks) {
        // stage slot_ks % 4 gets step slot_ks's data; a step past the row's
        // last (issued ahead, never read) reloads the last step, so no copy
        // addresses memory past the rows
        uint8_t *st = lds + (slot_ks & (G8NST - 1)) * L8::STAGE;
        const int ks = min(slot_ks, nk - 1);
        const int g = ks >> 2, s = ks & 3;
        const int wsoff = (g * 17 + 4 * s) * 128;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int q = 2 * wave + i;
            buf_to_lds16(ra, st + L8::ACT + 1024 * q, aoff[i], ks * G8K);
            buf_to_lds16(rw, st + L8::W + 1024 * q, woff[i], wsoff);
        }
        // the two gathers: wave 0 -> d_x block 0 (both row halves), wave 1 ->
        // d_x block 1, wave 2 -> d_w, wave 3 -> pad
        const int gsoff = wave < 2 ? ks * 8 : wave < 3 ? g * 17 * 128 + 4 * s : 0;
        buf_to_lds4(wave < 2 ? rdx : rw, st + (gdst0 - lds), goff[0], gsoff);
        buf_to_lds4(wave < 2 ? rdx : rw, st + (gdst0 - lds) + 256, goff[1], gsoff);
    };
    auto afrag = [&](const uint8_t *st, int R, int s2) {  // 16 k-bytes of activation row R, block s2, half h
        const int C = 2 * s2 + h;
        return *(const v4i *)(st + L8::ACT + R * G8K + 16 * (C ^ ((R >> 2) & 3)));
    };
    auto bfrag = [&](const uint8_t *st, int Cn, int s2) {  // 16 k-bytes of weight row Cn, block s2, half h
        const int piece = 2 * s2 + h;
        return *(const v4i *)(st + L8::W + ((Cn >> 3) * 4 + piece) * 128 + (Cn & 7) * 16);
    };

    v16i c0;
#pragma unroll
    for (int r = 0; r < 16; r++) c0[r] = C0;
    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // The copies are issued even for the steps a split never reaches (their
    // data is not read), so every wavefront's vmcnt stays exact.
    issue(ks0);
    issue(ks0 + 1);
    issue(ks0 + 2);
    for (int ks = ks0; ks < ks1; ks++) {
        wait_vmcnt<2 * G8COPIES>();  // this step's copies have landed (two later steps' may be in flight)
        stage_barrier();             // ... for every wavefront; and step ks - 1's stage is free
        issue(ks + 3);
        const uint8_t *st = lds + (ks & (G8NST - 1)) * L8::STAGE;
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            const int blk = 2 * ks + s2;
            if (blk >= p.nb) break;  // k an odd number of blocks: the last step's second block is padding
            v4i af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                af[t] = afrag(st, 64 * wm + 32 * t + l32, s2);
                bf[t] = bfrag(st, 64 * wn + 32 * t + l32, s2);
            }
            v16i D[2][2];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) D[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], c0, 0, 0, 0);
            float dw[2], ndw[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t pr = *(const uint32_t *)(st + L8::DW + 4 * (64 * wn + 32 * j + l32));
                dw[j] = f16_bits_to_f32(s2 ? pr >> 16 : pr & 0xffff);
                ndw[j] = -C0F * dw[j];
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                float dx[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4f v = *(const v4f *)(st + L8::DX + s2 * (G8T * 4) + 4 * (64 * wm + 32 * i + 8 * q + 4 * h));
                    dx[4 * q] = v.x;
                    dx[4 * q + 1] = v.y;
                    dx[4 * q + 2] = v.z;
                    dx[4 * q + 3] = v.w;
                }
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float t = __builtin_fmaf(u32_as_f32((uint32_t)D[i][j][r]), dw[j], ndw[j]);
                        acc[i][j][r] = __builtin_fmaf(t, dx[r], acc[i][j][r]);
                    }
            }
            if (DUMP) {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int col = n0 + 64 * wn + 32 * j + l32;
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int row = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                            if (row < p.m && col < p.n) {
                                const int64_t o = ((int64_t)row * p.n + col) * p.nb + blk;
                                p.S[o] = D[i][j][r] - C0;
                                p.Smin[o] = 0;
                            }
                        }
                    }
            }
        }
    }
    wait_vmcnt<0>();  // no copy may still be landing when the workgroup ends

    if (p.splits == 1) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + 64 * wn + 32 * j + l32;
            if (col >= p.n) continue;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < p.m) p.y[(int64_t)row * p.n + col] = acc[i][j][r];
                }
        }
        return;
    }
    // split-K: this partial tile, [128 rows][128 columns], summed by the reduce launch
    float *mine = p.part + ((int64_t)tile * p.splits + split) * (G8T * G8T);
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                mine[(64 * wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3)) * G8T + 64 * wn + 32 * j + l32] = acc[i][j][r];
}

struct Gemm8Plan {
    int ntm, ntn, tiles, splits, kss;
    size_t ws;
};

// Split K (halves, quarters, ...) while there are fewer work items than two
// per CU, each split keeping at least four steps.
Gemm8Plan gemm8_plan(int64_t m, int64_t n, int64_t k) {
    Gemm8Plan g;
    const int nk = (int)((k / QK8_0 + 1) / 2);
    g.ntm = (int)((m + G8T - 1) / G8T);
    g.ntn = (int)((n + G8T - 1) / G8T);
    g.tiles = g.ntm * g.ntn;
    g.splits = 1;
    while ((int64_t)g.tiles * g.splits < TARGET_WG8 && nk / (2 * g.splits) >= 4) g.splits *= 2;
    g.kss = (nk + g.splits - 1) / g.splits;
    g.splits = (nk + g.kss - 1) / g.kss;
    g.ws = g.splits > 1 ? (size_t)g.tiles * g.splits * G8T * G8T * 4 : 0;
    return g;
}

// Rows per launch: the copies address the activation quants with 32-bit
// offsets (rows * k < 2^31); longer inputs run as several launches.
int64_t gemm8_chunk_rows(int64_t m, int64_t k) {
    const int64_t cap = (((int64_t)1 << 31) - 1) / k / G8T * G8T;
    return m < cap ? m : cap;
}

}  // namespace

size_t gemm8_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % QK8_0 || k > (1 << 24)) return (size_t)-1;
    const int64_t mc = gemm8_chunk_rows(m, k);
    if (mc <= 0) return (size_t)-1;
    const Gemm8Plan g = gemm8_plan(mc, n, k);
    if (g.tiles > GEMM_MAX_TILES) return (size_t)-1;
    size_t ws = g.ws;
    if (m % mc) ws = std::max(ws, gemm8_plan(m % mc, n, k).ws);  // the last, shorter launch
    return ws;
}

hipError_t launch_gemm8(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                        int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s) {
    if (w.type != TYPE_Q8_0) return hipErrorNotSupported;
    if (!w.slab || !y || !x.qs || !x.d || m <= 0 || n <= 0 || k <= 0 || k % QK8_0) return hipErrorInvalidValue;
    if (m > 0x7fffffff || n > 0x7fffffff || k > (1 << 24) || w.ng != groups_of(TYPE_Q8_0, k)) return hipErrorInvalidValue;
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    // one n-tile's weights, addressed with 32-bit offsets
    if ((int64_t)(G8T / 8) * w.rb_stride >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    const int64_t mc = gemm8_chunk_rows(m, k);
    const int nb = (int)(k / QK8_0);
    for (int64_t r0 = 0; r0 < m; r0 += mc) {
        const int64_t mm = std::min(mc, m - r0);
        const Gemm8Plan g = gemm8_plan(mm, n, k);
        if (g.tiles > GEMM_MAX_TILES) return hipErrorNotSupported;
        if (g.splits > 1 && (!ws || ws_bytes < g.ws)) return hipErrorInvalidValue;
        Gemm8Params p;
        p.w = w.slab;
        p.rb_stride = w.rb_stride;
        p.ng = w.ng;
        p.xq = x.qs + r0 * k;
        p.xd = x.d + r0 * nb;
        p.y = y + r0 * n;
        p.part = (float *)ws;
        p.S = S ? S + r0 * n * nb : nullptr;
        p.Smin = Smin ? Smin + r0 * n * nb : nullptr;
        p.m = (int)mm;
        p.n = (int)n;
        p.k = (int)k;
        p.nb = nb;
        p.ntm = g.ntm;
        p.tiles = g.tiles;
        p.splits = g.splits;
        p.kss = g.kss;
        p.items = g.tiles * g.splits;
        p.per_xcd = (p.items + G8XCD - 1) / G8XCD;
        const unsigned grid = (unsigned)(p.per_xcd * G8XCD);
        if (S) gemm_q80_kernel<true><<<grid, 256, 0, s>>>(p);
        else gemm_q80_kernel<false><<<grid, 256, 0, s>>>(p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (g.splits > 1 && (e = launch_splitk_reduce(p.part, p.y, p.m, p.n, g.ntm, G8T, g.splits, g.tiles, s)) != hipSuccess)
            return e;
    }
    return hipSuccess;
}

}  // namespace aq
