// k_gemm6.hip -- prefill GEMM (m > 8) for Q6_K and Q5_K weights on the f16
// matrix cores, gfx950.
//
// Replaces the M-row loop of candle-core 0.8.4 k_quants::matmul<BlockQ6K> at
// prefill (native/arm_ai_nif/src/llama_candle.rs:93): for TinyLlama Q4_K_M
// these are attn_v and half of ffn_down.  Per super-block b of a weight row n
// and an activation row m (Q8_K):
//   y[m][n] += d_w[n,b] * d_x[m,b] * S,  S = sum_j sc_j * sum_{e in j} (q6_e - 32) * qx_e
// over the 16 sub-blocks j of 16 elements, with S an exact integer (candle's
// vec_dot keeps it exact too).
//
// Exactness on f16 MFMA.  Q6_K sub-scales use the whole int8 range
// (llama.cpp's quantizer maps the largest sub-block scale to -128), so
// sc_j * (q6_e - 32) reaches 128 * 32 = 4096 and is not exact in f16 (odd
// integers above 2048).  Each scale is split into two digits, sc = 16 * sh +
// sl with sh = sc >> 4 in -8..7 and sl = sc & 15 in 0..15, and the weight
// operand is built twice: w_h = sh * (q6 - 32) (|w_h| <= 256) and w_l = sl *
// (q6 - 32) (|w_l| <= 480), both integers exact in f16; the activation
// operand is the Q8_K quant qx (|qx| <= 128), exact in f16.  Each
// v_mfma_f32_32x32x16_f16 covers one sub-block (K = 16); products are exact in
// f32, and the two accumulator chains over all 16 sub-blocks of a super-block
// hold exact integers whatever the summation order: |A_h| <= 256 * 256 * 128
// = 2^23 and |A_l| <= 480 * 256 * 128 < 2^24.  S = 16 A_h + A_l (in int32 for
// the integer dump; one fma in f32 for the output, exact while |S| < 2^24).
// Each digit operand is built per lane from the 6-bit quants: nibble of ql,
// two bits of qh, then 1024 + q as f16 bits (0x6400 | q) and one packed f16
// fma, (1024 + q) * s - 1056 * s for s = sh or sl, which is exact (the result
// is an integer of magnitude <= 480; 1056 * s has at most 9 significant bits).
//
// Tiling.  A workgroup (4 wavefronts, two workgroups per CU) owns a 64 (m) x
// 128 (n) output tile; wavefront w owns columns 32w..32w+31 and both 32-row
// MFMA tiles, so each weight operand it builds feeds two MFMAs.  The f16
// activation rows of the tile (written by the Q8_K quantizer when it runs in
// the same call, else by qs_to_f16_kernel) are copied global
// -> LDS (buffer loads into LDS) one super-block ahead, two stages, 16-byte
// chunks XOR-swizzled by row; each lane loads its own column's ql / qh / scale
// bytes straight into registers, also one super-block ahead.  Work items
// (tile, k-split) are dealt so that all m-tiles and k-splits of one n-tile run
// on one XCD.  Split-K partials are summed in split order by the Q4_K GEMM's
// reduce launch.
//
// Q5_K (candle-core 0.8.4 k_quants::matmul<BlockQ5K>).  Per super-block
//   y[m][n] += d_x * (d_w * S - dmin_w * Smin),
//   S    = sum_j sc_j * sum_{e in j} q5_e * qx_e   (8 sub-blocks of 32, q5 in 0..31)
//   Smin = sum_g bsums[m,g] * mn_{g/2}              (16 groups of 16)
// The weight operand sc_j * q5 <= 63 * 31 = 1953 is an integer exact in f16,
// built as (1024 + q5) * sc - 1024 * sc in one fma (one rounding, of an exact
// integer); every partial sum of two sub-blocks (64 elements) is at most
// 64 * 1953 * 128 < 2^24, so four accumulator chains of four MFMAs each hold
// exact integers, and S is their sum (exact in int32 for the dump; in f32 for
// the output).  Smin is one M x 16 by 16 x N f16 MFMA per super-block of
// bsums (|.| <= 2048, exact in f16) and mins (<= 63), every partial sum below
// 16 * 2048 * 63 < 2^24, so exact.  Piece 0 of the group (d, dmin, the twelve
// packed scale bytes) is loaded whole by each lane; the bsums rows of the tile
// are copied into LDS beside the quants.
#include "gemm6_impl.h"

namespace aq {

size_t gemm6_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % QK_K || k > (1 << 24)) return (size_t)-1;
    const int64_t mc = std::min(m, gemm6_chunk_rows(k));
    if (mc <= 0) return (size_t)-1;
    Gemm6Plan g = gemm6_plan(mc, n, k);
    if (g.tiles > GEMM_MAX_TILES) return (size_t)-1;
    size_t ws = g.ws;
    if (m % mc) ws = std::max(ws, gemm6_plan(m % mc, n, k).ws);
    return ws;
}

hipError_t launch_gemm6(const WLayout &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y, int32_t *S,
                        int32_t *Smin, void *ws, size_t ws_bytes, hipStream_t s) {
    if (w.type != TYPE_Q6_K && w.type != TYPE_Q5_K) return hipErrorNotSupported;
    const bool q5 = w.type == TYPE_Q5_K;
    if (!w.slab || (!q5 && !w.d) || (q5 && !x.bsum16) || !y || !x.qs || !x.d || m <= 0 || n <= 0 || k <= 0 || k % QK_K)
        return hipErrorInvalidValue;
    if (m > 0x7fffffff || n > 0x7fffffff || k > (1 << 24) || w.ng != k / QK_K) return hipErrorInvalidValue;
    if ((int64_t)16 * w.rb_stride >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    const int64_t mc = std::min(m, gemm6_chunk_rows(k));
    if (mc <= 0) return hipErrorNotSupported;
    const int ng = w.ng;
    for (int64_t r0 = 0; r0 < m; r0 += mc) {
        const int64_t mm = std::min(mc, m - r0);
        const Gemm6Plan g = gemm6_plan(mm, n, k);
        if (g.tiles > GEMM_MAX_TILES) return hipErrorNotSupported;
        if (!ws || ws_bytes < g.ws) return hipErrorInvalidValue;
        // the quants as f16: the activation's own plane when its quantizer
        // wrote one, else converted into the workspace here
        uint16_t *x16 = x.q16 ? x.q16 + r0 * k : (uint16_t *)((uint8_t *)ws + align_up(g.part, 256));
        hipError_t e;
        if (!x.q16) {
            const int64_t n4 = mm * k / 4;
            qs_to_f16_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>(x.qs + r0 * k, n4, x16);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        Gemm6Params p;
        p.w = w.slab;
        p.wd = w.d;
        p.rb_stride = w.rb_stride;
        p.ng = ng;
        p.x16 = x16;
        p.xd = x.d + r0 * ng;
        p.xbs = q5 ? x.bsum16 + r0 * (k / 16) : nullptr;
        p.y = y + r0 * n;
        p.m = (int)mm;
        p.n = (int)n;
        p.k = (int)k;
        p.ntm = g.ntm;
        p.tiles = g.tiles;
        p.splits = g.splits;
        p.kbs = g.kbs;
        p.items = g.tiles * g.splits;
        p.per_xcd = (p.items + NXCD6 - 1) / NXCD6;
        p.part = (float *)ws;
        p.S = S ? S + r0 * n * ng : nullptr;
        p.Smin = Smin ? Smin + r0 * n * ng : nullptr;
        const unsigned grid = (unsigned)(p.per_xcd * NXCD6);
        if (q5) {
            if (S) gemm_f16w_kernel<TYPE_Q5_K, true><<<grid, 256, 0, s>>>(p);
            else gemm_f16w_kernel<TYPE_Q5_K, false><<<grid, 256, 0, s>>>(p);
        } else {
            if (S) gemm_f16w_kernel<TYPE_Q6_K, true><<<grid, 256, 0, s>>>(p);
            else gemm_f16w_kernel<TYPE_Q6_K, false><<<grid, 256, 0, s>>>(p);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (g.splits > 1) {
            e = launch_splitk_reduce(p.part, p.y, p.m, p.n, g.ntm, G6M, g.splits, g.tiles, s);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace aq
