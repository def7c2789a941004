// k_matvec.hip -- decode-path matvec (batch 1..8) for Q4_K / Q6_K / Q8_0
// weights against Q8_K / Q8_0 activations, gfx950.
//
// Replaces the column loop of candle-core 0.8.4 k_quants::matmul<T> (each
// output column = T::vec_dot(k, W[col], xq[row])), reached from
// native/arm_ai_nif/src/llama_candle.rs:119 at decode.  The integer part of
// every block dot product is computed exactly (v_dot4_i32_i8 on 4 bytes at a
// time); only the f32 combination order differs from candle's vec_dot_unopt.
//
// Mapping.  A weight row is cut into "chunks" of 16 B of Q4_K quants (32
// elements), 48 B of Q6_K quants (64 elements) or one 32-element Q8_0
// block.  A row group of wpr wavefronts (64*wpr threads) owns a row at a
// time; thread t owns chunks t, t+64*wpr, ... (CPL of them), so its slice of
// the activation (all B batch rows) is loaded into registers once and reused
// for every weight row the group visits.  Weight loads are 128-bit and
// coalesced: consecutive lanes read consecutive 16 B of the same row.  The
// per-thread partial sums are reduced with DPP row ops and readlane, and
// through LDS across the waves of a row group.
#include "aq_internal.h"

namespace aq {

struct MvArgs {
    WPlanes w;
    ActPlanes x;  // already offset to the first activation row of the slice
    float *y;     // already offset; row stride n
    int32_t *S;   // integer dump (or null), already offset; [m][n][nblk]
    int32_t *Smin;
    int n, k, m;  // m = rows in this slice (<= B)
    int rows_per_group;
    int wpr;
};

// ------------------------------------------------------------------ Q4_K
struct FmtQ4K {
    static constexpr int ELEMS = 32, CPB = 8, LOG_CPB = 3, BLK = 256, REGS = 11;
    struct Act {
        int lo[4], hi[4];
        int bs_lo, bs_hi;
        float d;
    };
    struct Wt {
        uint4 q, meta;
    };
    // chunk c: super-block sb = c/8, piece p = c%8 = (cc, h): 16 bytes
    // qs[32cc+16h ..] hold elements 64cc+16h+i (low nibble, sub-block 2cc)
    // and 64cc+32+16h+i (high nibble, sub-block 2cc+1).
    __device__ static void load_act(Act &A, const ActPlanes &x, int row, int c, int k) {
        const int sb = c >> 3, p = c & 7, cc = p >> 1, h = p & 1;
        const int8_t *xr = x.qs + (size_t)row * k + sb * 256 + 64 * cc + 16 * h;
        const int4 v0 = *(const int4 *)xr, v1 = *(const int4 *)(xr + 32);
        A.lo[0] = v0.x; A.lo[1] = v0.y; A.lo[2] = v0.z; A.lo[3] = v0.w;
        A.hi[0] = v1.x; A.hi[1] = v1.y; A.hi[2] = v1.z; A.hi[3] = v1.w;
        const int16_t *bs = x.bsums + (size_t)row * (k / 16) + sb * 16 + 4 * cc + h;
        A.bs_lo = bs[0];
        A.bs_hi = bs[2];
        A.d = x.d[(size_t)row * (k / 256) + sb];
    }
    __device__ static void load_w(Wt &W, const WPlanes &w, int64_t row, int c, int k) {
        W.q = *(const uint4 *)(w.qs + row * (k / 2) + (int64_t)c * 16);
        W.meta = *(const uint4 *)(w.meta + (row * (k / 256) + (c >> 3)) * 16);
    }
    __device__ static void dot1(const Wt &W, int pos, const Act *A, int B, int *S, int *Smin, float *f);
};

template <int B>
__device__ __forceinline__ void q4k_dot(const FmtQ4K::Wt &W, int pos, const FmtQ4K::Act (&A)[B], int (&S)[B],
                                        int (&Smin)[B], float (&f)[B]) {
    const uint32_t q[4] = {W.q.x, W.q.y, W.q.z, W.q.w};
    int lo4[4], hi4[4];
    for (int i = 0; i < 4; i++) {
        lo4[i] = (int)(q[i] & 0x0F0F0F0Fu);
        hi4[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
    }
    // 6-bit scales / mins of the super-block (candle's utmp form of
    // GGML get_scale_min_k4): words of four bytes each.
    const uint32_t u0 = W.meta.y, u1 = W.meta.z, u2 = W.meta.w;
    const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
    const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
    const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const int cc = pos >> 1;
    const uint32_t sw = cc < 2 ? sc03 : sc47, mw = cc < 2 ? mn03 : mn47;
    const int sh = (cc & 1) * 16;
    const int sc_lo = (sw >> sh) & 0xff, sc_hi = (sw >> (sh + 8)) & 0xff;
    const int m_lo = (mw >> sh) & 0xff, m_hi = (mw >> (sh + 8)) & 0xff;
    const float dw = f16_bits_to_f32(W.meta.x), dmw = f16_bits_to_f32(W.meta.x >> 16);
#pragma unroll
    for (int b = 0; b < B; b++) {
        int il = 0, ih = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            il = sdot4(lo4[i], A[b].lo[i], il);
            ih = sdot4(hi4[i], A[b].hi[i], ih);
        }
        S[b] = sc_lo * il + sc_hi * ih;
        Smin[b] = m_lo * A[b].bs_lo + m_hi * A[b].bs_hi;
        f[b] = (float)S[b] * (dw * A[b].d) - (float)Smin[b] * (dmw * A[b].d);
    }
}

// ------------------------------------------------------------------ Q6_K
struct FmtQ6K {
    static constexpr int ELEMS = 64, CPB = 4, LOG_CPB = 2, BLK = 256, REGS = 21;
    struct Act {
        int x[4][4];  // [g][word]
        int bs[4];
        float d;
    };
    struct Wt {
        uint4 a, b, h, sc;
        uint32_t d;
    };
    // chunk c: super-block sb = c/4, q = c%4 = (hh, l0 = 16*(q&1)); group g
    // covers elements 128hh + 32g + l0 + i, sub-block 8hh + 2g + (q&1).
    __device__ static void load_act(Act &A, const ActPlanes &x, int row, int c, int k) {
        const int sb = c >> 2, q = c & 3, hh = q >> 1, odd = q & 1;
        const int8_t *xr = x.qs + (size_t)row * k + sb * 256 + 128 * hh + 16 * odd;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int4 v = *(const int4 *)(xr + 32 * g);
            A.x[g][0] = v.x; A.x[g][1] = v.y; A.x[g][2] = v.z; A.x[g][3] = v.w;
        }
        const int16_t *bs = x.bsums + (size_t)row * (k / 16) + sb * 16 + 8 * hh + odd;
#pragma unroll
        for (int g = 0; g < 4; g++) A.bs[g] = bs[2 * g];
        A.d = x.d[(size_t)row * (k / 256) + sb];
    }
    __device__ static void load_w(Wt &W, const WPlanes &w, int64_t row, int c, int k) {
        const int64_t blk = row * (k / 256) + (c >> 2);
        const int q = c & 3;
        const uint8_t *ql = w.qs + blk * 128 + 32 * q;
        W.a = *(const uint4 *)ql;
        W.b = *(const uint4 *)(ql + 16);
        W.h = *(const uint4 *)(w.qh + blk * 64 + 16 * q);
        W.sc = *(const uint4 *)(w.meta + blk * 16);
        W.d = w.d[blk];
    }
};

template <int B>
__device__ __forceinline__ void q6k_dot(const FmtQ6K::Wt &W, int pos, const FmtQ6K::Act (&A)[B], int (&S)[B],
                                        int (&Smin)[B], float (&f)[B]) {
    const uint32_t a[4] = {W.a.x, W.a.y, W.a.z, W.a.w};
    const uint32_t bq[4] = {W.b.x, W.b.y, W.b.z, W.b.w};
    const uint32_t h[4] = {W.h.x, W.h.y, W.h.z, W.h.w};
    int q[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        q[0][i] = (int)((a[i] & 0x0F0F0F0Fu) | ((h[i] << 4) & 0x30303030u));
        q[1][i] = (int)((bq[i] & 0x0F0F0F0Fu) | ((h[i] << 2) & 0x30303030u));
        q[2][i] = (int)(((a[i] >> 4) & 0x0F0F0F0Fu) | (h[i] & 0x30303030u));
        q[3][i] = (int)(((bq[i] >> 4) & 0x0F0F0F0Fu) | ((h[i] >> 2) & 0x30303030u));
    }
    // sub-scales 8hh + 2g + odd: word 2hh + g/2, byte 2(g&1) + odd
    const int hh = pos >> 1, odd = pos & 1;
    const uint32_t w0 = hh ? W.sc.z : W.sc.x, w1 = hh ? W.sc.w : W.sc.y;
    int sc[4];
    sc[0] = (int)(int8_t)(w0 >> (8 * odd));
    sc[1] = (int)(int8_t)(w0 >> (8 * (2 + odd)));
    sc[2] = (int)(int8_t)(w1 >> (8 * odd));
    sc[3] = (int)(int8_t)(w1 >> (8 * (2 + odd)));
    const float dw = f16_bits_to_f32(W.d);
#pragma unroll
    for (int b = 0; b < B; b++) {
        int s = 0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int t = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) t = sdot4(q[g][i], A[b].x[g][i], t);
            // sum (q6 - 32) * x = sum q6 * x - 32 * bsum (bsum = sum of the same 16 x)
            s += sc[g] * (t - 32 * A[b].bs[g]);
        }
        S[b] = s;
        Smin[b] = 0;
        f[b] = (float)s * (dw * A[b].d);
    }
}

// ------------------------------------------------------------------ Q8_0
struct FmtQ80 {
    static constexpr int ELEMS = 32, CPB = 1, LOG_CPB = 0, BLK = 32, REGS = 9;
    struct Act {
        int x[8];
        float d;
    };
    struct Wt {
        uint4 a, b;
        uint32_t d;
    };
    __device__ static void load_act(Act &A, const ActPlanes &x, int row, int c, int k) {
        const int8_t *xr = x.qs + (size_t)row * k + (size_t)c * 32;
        const int4 v0 = *(const int4 *)xr, v1 = *(const int4 *)(xr + 16);
        A.x[0] = v0.x; A.x[1] = v0.y; A.x[2] = v0.z; A.x[3] = v0.w;
        A.x[4] = v1.x; A.x[5] = v1.y; A.x[6] = v1.z; A.x[7] = v1.w;
        A.d = x.d[(size_t)row * (k / 32) + c];
    }
    __device__ static void load_w(Wt &W, const WPlanes &w, int64_t row, int c, int k) {
        const uint8_t *p = w.qs + row * k + (int64_t)c * 32;
        W.a = *(const uint4 *)p;
        W.b = *(const uint4 *)(p + 16);
        W.d = w.d[row * (k / 32) + c];
    }
};

template <int B>
__device__ __forceinline__ void q80_dot(const FmtQ80::Wt &W, int, const FmtQ80::Act (&A)[B], int (&S)[B],
                                        int (&Smin)[B], float (&f)[B]) {
    const int w[8] = {(int)W.a.x, (int)W.a.y, (int)W.a.z, (int)W.a.w,
                      (int)W.b.x, (int)W.b.y, (int)W.b.z, (int)W.b.w};
    const float dw = f16_bits_to_f32(W.d);
#pragma unroll
    for (int b = 0; b < B; b++) {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) s = sdot4(w[i], A[b].x[i], s);
        S[b] = s;
        Smin[b] = 0;
        // candle: sumf += (sum_i as f32) * f16(d_w) * f16(d_x), left to right
        f[b] = ((float)s * dw) * A[b].d;
    }
}

template <class F, int B>
__device__ __forceinline__ void fmt_dot(const typename F::Wt &W, int pos, const typename F::Act (&A)[B],
                                        int (&S)[B], int (&Smin)[B], float (&f)[B]) {
    if constexpr (F::BLK == 256 && F::CPB == 8) q4k_dot<B>(W, pos, A, S, Smin, f);
    else if constexpr (F::CPB == 4) q6k_dot<B>(W, pos, A, S, Smin, f);
    else q80_dot<B>(W, pos, A, S, Smin, f);
}

// ----------------------------------------------------------------- kernel
template <class F, int B, int CPL, bool DUMP>
__global__ __launch_bounds__(256) void matvec_kernel(MvArgs a) {
    __shared__ float red[4][B];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wpr = a.wpr, G = 4 / wpr;
    const int grp = wave / wpr, wig = wave - grp * wpr;
    const int T = 64 * wpr, t = wig * 64 + lane;
    const int C = a.k / F::ELEMS;
    const int pos = t & (F::CPB - 1);  // T is a multiple of CPB, so pos is the same for all chunks
    const int nblk = a.k / F::BLK;

    typename F::Act act[CPL][B];
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = t + T * i;
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (c < C) F::load_act(act[i][b], a.x, b < a.m ? b : 0, c, a.k);
            else act[i][b] = typename F::Act{};
        }
    }

    const int64_t row0 = ((int64_t)blockIdx.x * G + grp) * a.rows_per_group;
    for (int r = 0; r < a.rows_per_group; r++) {
        const int64_t row = row0 + r;
        const bool rv = row < a.n;  // uniform over the row group
        float acc[B];
#pragma unroll
        for (int b = 0; b < B; b++) acc[b] = 0.0f;
        typename F::Wt wt[CPL];
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            const int c = t + T * i;
            if (rv && c < C) F::load_w(wt[i], a.w, row, c, a.k);
            else wt[i] = typename F::Wt{};
        }
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            int S[B], Sm[B];
            float f[B];
            fmt_dot<F, B>(wt[i], pos, act[i], S, Sm, f);
#pragma unroll
            for (int b = 0; b < B; b++) acc[b] += f[b];
            if constexpr (DUMP) {
                const int c = t + T * i;
#pragma unroll
                for (int b = 0; b < B; b++) {
                    const int s = group_sum_i<F::LOG_CPB>(S[b]);
                    const int sm = group_sum_i<F::LOG_CPB>(Sm[b]);
                    if (rv && c < C && pos == 0 && b < a.m) {
                        const int64_t o = ((int64_t)b * a.n + row) * nblk + c / F::CPB;
                        a.S[o] = s;
                        a.Smin[o] = sm;
                    }
                }
            }
        }
#pragma unroll
        for (int b = 0; b < B; b++) acc[b] = wave_sum(acc[b]);
        if (wpr == 1) {
#pragma unroll
            for (int b = 0; b < B; b++)
                if (lane == b && rv && b < a.m) a.y[(int64_t)b * a.n + row] = acc[b];
        } else {
            if (lane == 0) {
#pragma unroll
                for (int b = 0; b < B; b++) red[wave][b] = acc[b];
            }
            __syncthreads();
            if (wig == 0 && lane < B && lane < a.m && rv) {
                float s = 0.0f;
                for (int j = 0; j < wpr; j++) s += red[grp * wpr + j][lane];
                a.y[(int64_t)lane * a.n + row] = s;
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------- host
namespace {

constexpr int REG_BUDGET = 96;  // activation registers per thread

template <class F>
constexpr bool feasible(int B, int CPL) {
    return B * CPL * F::REGS <= REG_BUDGET;
}

template <class F, int B, int CPL>
hipError_t launch_one(const MvArgs &a, unsigned grid, bool dump, hipStream_t s) {
    if constexpr (feasible<F>(B, CPL)) {
        if (dump) matvec_kernel<F, B, CPL, true><<<grid, 256, 0, s>>>(a);
        else matvec_kernel<F, B, CPL, false><<<grid, 256, 0, s>>>(a);
        return hipGetLastError();
    } else {
        return hipErrorInvalidConfiguration;
    }
}

template <class F, int B>
hipError_t launch_cpl(int cpl, const MvArgs &a, unsigned grid, bool dump, hipStream_t s) {
    switch (cpl) {
    case 1: return launch_one<F, B, 1>(a, grid, dump, s);
    case 2: return launch_one<F, B, 2>(a, grid, dump, s);
    case 4: return launch_one<F, B, 4>(a, grid, dump, s);
    case 8: return launch_one<F, B, 8>(a, grid, dump, s);
    default: return hipErrorInvalidConfiguration;
    }
}

template <class F>
hipError_t launch_b(int B, int cpl, const MvArgs &a, unsigned grid, bool dump, hipStream_t s) {
    switch (B) {
    case 1: return launch_cpl<F, 1>(cpl, a, grid, dump, s);
    case 2: return launch_cpl<F, 2>(cpl, a, grid, dump, s);
    case 4: return launch_cpl<F, 4>(cpl, a, grid, dump, s);
    case 8: return launch_cpl<F, 8>(cpl, a, grid, dump, s);
    default: return hipErrorInvalidConfiguration;
    }
}

// Smallest (wpr, cpl) with wpr*64*cpl >= C chunks within the register budget.
template <class F>
bool pick_config(int B, int C, int *wpr_out, int *cpl_out) {
    for (int wpr = 1; wpr <= 4; wpr *= 2)
        for (int cpl = 1; cpl <= 8; cpl *= 2)
            if (B * cpl * F::REGS <= REG_BUDGET && wpr * 64 * cpl >= C) {
                *wpr_out = wpr;
                *cpl_out = cpl;
                return true;
            }
    return false;
}

template <class F>
hipError_t launch_type(const WPlanes &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m, float *y,
                       int32_t *S, int32_t *Smin, hipStream_t s) {
    if (k % F::BLK || n <= 0 || n > 0x7fffffff || k > 0x7fffffff) return hipErrorInvalidValue;
    const int C = (int)(k / F::ELEMS);
    const int64_t nblk = k / F::BLK;
    const bool dump = S != nullptr;
    int64_t r0 = 0;
    while (r0 < m) {
        const int64_t rem = m - r0;
        int B = rem >= 8 ? 8 : rem >= 4 ? 4 : rem >= 2 ? 2 : 1;
        if (rem == 3) B = 4;
        if (rem > 4 && rem < 8) B = 8;
        int wpr = 0, cpl = 0;
        while (!pick_config<F>(B, C, &wpr, &cpl)) {
            if (B == 1) return hipErrorNotSupported;  // k too large for one pass
            B /= 2;
        }
        const int mb = (int)(rem < B ? rem : B);
        MvArgs a;
        a.w = w;
        a.x.qs = x.qs + r0 * k;
        a.x.d = x.d + r0 * (k / (F::BLK == 32 ? 32 : 256));
        a.x.d16 = x.d16;
        a.x.bsums = x.bsums + r0 * (k / 16);
        a.y = y + r0 * n;
        a.S = dump ? S + r0 * n * nblk : nullptr;
        a.Smin = dump ? Smin + r0 * n * nblk : nullptr;
        a.n = (int)n;
        a.k = (int)k;
        a.m = mb;
        a.wpr = wpr;
        // About 4096 wavefronts in flight; each row group walks rows_per_group rows.
        const int64_t groups_target = (4096 + wpr - 1) / wpr;
        int rpg = (int)((n + groups_target - 1) / groups_target);
        if (rpg < 1) rpg = 1;
        a.rows_per_group = rpg;
        const int G = 4 / wpr;
        const int64_t groups = (n + rpg - 1) / rpg;
        const int64_t grid = (groups + G - 1) / G;
        if (grid > 0x7fffffff) return hipErrorInvalidValue;
        hipError_t e = launch_b<F>(B, cpl, a, (unsigned)grid, dump, s);
        if (e != hipSuccess) return e;
        r0 += mb;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_matvec(int type, const WPlanes &w, int64_t n, int64_t k, const ActPlanes &x, int64_t m,
                         float *y, int32_t *S, int32_t *Smin, hipStream_t s) {
    if (m < 0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    switch (type) {
    case TYPE_Q4_K: return launch_type<FmtQ4K>(w, n, k, x, m, y, S, Smin, s);
    case TYPE_Q6_K: return launch_type<FmtQ6K>(w, n, k, x, m, y, S, Smin, s);
    case TYPE_Q8_0: return launch_type<FmtQ80>(w, n, k, x, m, y, S, Smin, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace aq
