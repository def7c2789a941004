// k_matvec.hip -- decode-path matvec (batch 1..8 per pass) for Q4_K / Q6_K /
// Q8_0 weights against Q8_K / Q8_0 activations, gfx950.
//
// Replaces the column loop of candle-core 0.8.4 k_quants::matmul<T> (each
// output column = T::vec_dot(k, W[col], xq[row])), reached from
// native/arm_ai_nif/src/llama_candle.rs:119 at decode.  The integer part of
// every block dot product is computed exactly (v_dot4_i32_i8 on 4 bytes at a
// time); only the f32 combination order differs from candle's vec_dot_unopt.
//
// Mapping.  A wavefront works on one 8-row block of the weight (the
// row-block tile layout of aq_internal.h) and a chunk of 8 of its 256-element
// groups: lane (g_l, r_l) = (lane / 8, lane % 8) owns group 8*chunk + g_l of
// row 8*block + r_l, so each 16-byte load instruction of the wavefront reads
// eight full 128-byte lines (nontemporal: the weights are read once per call).
// A workgroup iteration covers rbw = max(1, 8 / chunks) row blocks with
// nw = min(8, rbw * chunks) wavefronts (no idle wavefronts below 8 chunks; above
// 8, wavefront w takes chunks w, w + 8, ...).  A row's chunk partials are
// reduced across the chunk's lanes (butterfly) and across wavefronts through
// LDS, in chunk order.  Each wavefront prefetches its next step's weights
// before computing the current one (ping-pong registers).  The activation (all batch rows of the
// pass) sits in LDS as one 304-byte record per (row, group); the records'
// stride spreads the 16-byte reads of consecutive lanes over disjoint LDS
// banks.  With an f32 input the workgroup quantises it into LDS itself (same
// device code as the quantizer kernels, so the same bytes) while its first
// weight loads are in flight.
#include "aq_internal.h"

#include <mutex>

namespace aq {

namespace {

constexpr int REC = 304;           // LDS bytes per (batch row, group) activation record
constexpr int REC_BSUMS = 256;     // Q8_K record: i16 bsums[16]
constexpr int REC_D = 288;         // Q8_K record: f32 d
constexpr int REC_D8 = 256;        // Q8_0 record: f32 d[8] (value of the f16 d)
constexpr size_t LDS_CAP = 144 * 1024;  // activation records per workgroup (gfx950: 160 KB of LDS per CU)
constexpr int TARGET_WAVES = 8192;  // resident wavefronts aimed at: 32 per CU on 256 CUs
constexpr int MIN_WAVES = 1536;     // split a row block over wavefronts below this many

struct MvParams {
    const uint8_t *w;    // row-block tiles
    const uint16_t *wd;  // Q6_K d plane
    int64_t rb_stride;
    int n, k, ng, nch, np, rbw, nw, nsub, m, iters;  // np: wavefronts per row block, nsub: chunks per wavefront
    const float *x;      // fused: f32 [m][k] of this pass, or null
    // fused input transforms (m = 1; the XF template argument selects one):
    //   XF_NORM: quantise rms_norm(x + xdelta) * xnorm, and workgroup 0 writes
    //            x + xdelta to xout (xdelta, xout may be null);
    //   XF_SILU: x = [g (k) | u (k)]: quantise silu(g) * u.
    const float *xdelta, *xnorm;
    float *xout;
    float eps;
    ActPlanes act;       // pre-quantised planes of this pass (when x is null)
    float *y;            // [m][n] of this pass
    int32_t *S, *Smin;   // [m][n][blocks] of this pass, or null
};

template <int TYPE>
struct Wt {
    uint4 pc[slabs_of(TYPE)];
    uint32_t d;  // Q6_K super-block d (f16 bits); Q2_K d | dmin << 16
};

// Weights are streamed once per call: nontemporal loads keep them from
// displacing the (reused) activation in the caches.  Row block rb is
// wave-uniform; a row block past the end (or a group past the row) reads zeros.
template <int TYPE>
__device__ __forceinline__ void load_w(Wt<TYPE> &W, const MvParams &p, int rb, int nrb, int g, int r_l) {
    constexpr int S = slabs_of(TYPE);
    const bool rb_ok = rb < nrb;
    const rsrc_t r = buf_rsrc(p.w + (int64_t)rb * p.rb_stride, rb_ok ? (uint32_t)p.rb_stride : 0u);
    const uint32_t off = g < p.ng ? (uint32_t)(g * (S * 128) + r_l * 16) : BUF_OOB;
#pragma unroll
    for (int i = 0; i < S; i++) {
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, off + i * 128, 0, BUF_NT);
        W.pc[i] = make_uint4(t.x, t.y, t.z, t.w);
    }
    if (TYPE == TYPE_Q6_K) {
        const rsrc_t rd = buf_rsrc(p.wd + (int64_t)rb * p.ng * RB, rb_ok ? (uint32_t)(p.ng * RB * 2) : 0u);
        W.d = __builtin_amdgcn_raw_buffer_load_b16(rd, g < p.ng ? (uint32_t)((g * RB + r_l) * 2) : BUF_OOB, 0, BUF_NT);
    }
    if (TYPE == TYPE_Q2_K) {  // d | dmin << 16
        const rsrc_t rd = buf_rsrc(p.wd + (int64_t)rb * p.ng * RB * 2, rb_ok ? (uint32_t)(p.ng * RB * 4) : 0u);
        W.d = __builtin_amdgcn_raw_buffer_load_b32(rd, g < p.ng ? (uint32_t)((g * RB + r_l) * 4) : BUF_OOB, 0, BUF_NT);
    }
}

__device__ __forceinline__ int byte_u(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ int byte_s(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }
__device__ __forceinline__ int lo16(uint32_t w) { return (int)(int16_t)(w & 0xffffu); }
__device__ __forceinline__ int hi16(uint32_t w) { return (int)(int16_t)(w >> 16); }

__device__ __forceinline__ int dot16(const uint32_t q[4], const int4 x, int acc) {
    acc = sdot4((int)q[0], x.x, acc);
    acc = sdot4((int)q[1], x.y, acc);
    acc = sdot4((int)q[2], x.z, acc);
    acc = sdot4((int)q[3], x.w, acc);
    return acc;
}

// ------------------------------------------------------------ Q4_K, Q5_K
// Super-block: piece 0 = d, dmin, 12 scale bytes; piece QP + 2c + h = qs bytes
// 32c + 16h .. +15, whose low nibbles are elements 64c + 16h + i (sub-block
// 2c) and high nibbles elements 64c + 32 + 16h + i (sub-block 2c + 1).
// Q4_K: QP = 1.  Q5_K: QP = 3, pieces 1 + h = qh bytes 16h .. +15, and bit s
// of qh[l] is bit 4 of element 32s + l (bit 2c for the low nibbles of chunk
// c, bit 2c + 1 for its high nibbles).
template <int B, bool DUMP, int TYPE>
__device__ __forceinline__ void dot_q45k(const Wt<TYPE> &W, const uint8_t *lds, int ng, int g, int m,
                                         float (&f)[B], int (&So)[B], int (&Smo)[B]) {
    constexpr bool FIVE = TYPE == TYPE_Q5_K;
    constexpr int QP = FIVE ? 3 : 1;
    const uint32_t u0 = W.pc[0].y, u1 = W.pc[0].z, u2 = W.pc[0].w;
    // candle's utmp form of GGML get_scale_min_k4 (6-bit scales and mins)
    const uint32_t sc03 = u0 & 0x3F3F3F3Fu;
    const uint32_t sc47 = (u2 & 0x0F0F0F0Fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t mn03 = u1 & 0x3F3F3F3Fu;
    const uint32_t mn47 = ((u2 >> 4) & 0x0F0F0F0Fu) | (((u1 >> 6) & 0x03030303u) << 4);
    const float dw = f16_bits_to_f32(W.pc[0].x), dmw = f16_bits_to_f32(W.pc[0].x >> 16);
    int S[B];
#pragma unroll
    for (int b = 0; b < B; b++) S[b] = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        int il[B], ih[B];
#pragma unroll
        for (int b = 0; b < B; b++) il[b] = ih[b] = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint4 q = W.pc[QP + 2 * c + h];
            uint32_t lo[4] = {q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu};
            uint32_t hi[4] = {(q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                              (q.w >> 4) & 0x0F0F0F0Fu};
            if (FIVE) {
                const uint4 qh = W.pc[1 + h];
                const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    lo[i] |= ((hw[i] >> (2 * c)) & 0x01010101u) << 4;
                    hi[i] |= ((hw[i] >> (2 * c + 1)) & 0x01010101u) << 4;
                }
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                if (b < m) {
                    const uint8_t *rec = lds + (b * ng + g) * REC + 64 * c + 16 * h;
                    il[b] = dot16(lo, *(const int4 *)rec, il[b]);
                    ih[b] = dot16(hi, *(const int4 *)(rec + 32), ih[b]);
                }
            }
        }
        const uint32_t sw = c < 2 ? sc03 : sc47;
        const int s_lo = byte_u(sw, 2 * (c & 1)), s_hi = byte_u(sw, 2 * (c & 1) + 1);
#pragma unroll
        for (int b = 0; b < B; b++) S[b] += s_lo * il[b] + s_hi * ih[b];
    }
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const uint8_t *rec = lds + (b * ng + g) * REC;
            const int4 p0 = *(const int4 *)(rec + REC_BSUMS), p1 = *(const int4 *)(rec + REC_BSUMS + 16);
            // bsums dword j holds bsums[2j], bsums[2j+1]: the two halves of sub-block j
            const uint32_t pw[8] = {(uint32_t)p0.x, (uint32_t)p0.y, (uint32_t)p0.z, (uint32_t)p0.w,
                                    (uint32_t)p1.x, (uint32_t)p1.y, (uint32_t)p1.z, (uint32_t)p1.w};
            int smin = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int mj = byte_u(j < 4 ? mn03 : mn47, j & 3);
                smin += mj * (lo16(pw[j]) + hi16(pw[j]));
            }
            const float dx = *(const float *)(rec + REC_D);
            f[b] += (dw * dx) * (float)S[b] - (dmw * dx) * (float)smin;
            if (DUMP) {
                So[b] = S[b];
                Smo[b] = smin;
            }
        }
    }
}

// ------------------------------------------------------------------ Q6_K
// Super-block: pieces 0..7 = ql, 8..11 = qh, 12 = the 16 int8 sub-scales.
// For half hh and 16-element half t, pieces A = ql[4hh + t], Bq = ql[4hh + 2 + t]
// and H = qh[2hh + t] hold elements 128hh + 32gq + 16t + i (gq = 0..3):
//   gq0: A & 0xF | (H & 3) << 4        gq1: Bq & 0xF | (H >> 2 & 3) << 4
//   gq2: A >> 4 | (H >> 4 & 3) << 4    gq3: Bq >> 4 | (H >> 6 & 3) << 4
// each minus 32; sub-block of element e is e/16 = 8hh + 2gq + t.
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q6k(const Wt<TYPE_Q6_K> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], int (&So)[B], int (&Smo)[B]) {
    const uint32_t scw[4] = {W.pc[12].x, W.pc[12].y, W.pc[12].z, W.pc[12].w};
    int S[B];
#pragma unroll
    for (int b = 0; b < B; b++) S[b] = 0;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint4 A = W.pc[4 * hh + t], Bq = W.pc[4 * hh + 2 + t], H = W.pc[8 + 2 * hh + t];
            const uint32_t a[4] = {A.x, A.y, A.z, A.w}, bq[4] = {Bq.x, Bq.y, Bq.z, Bq.w}, hq[4] = {H.x, H.y, H.z, H.w};
            uint32_t q[4][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                q[0][i] = (a[i] & 0x0F0F0F0Fu) | ((hq[i] << 4) & 0x30303030u);
                q[1][i] = (bq[i] & 0x0F0F0F0Fu) | ((hq[i] << 2) & 0x30303030u);
                q[2][i] = ((a[i] >> 4) & 0x0F0F0F0Fu) | (hq[i] & 0x30303030u);
                q[3][i] = ((bq[i] >> 4) & 0x0F0F0F0Fu) | ((hq[i] >> 2) & 0x30303030u);
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                if (b < m) {
                    const uint8_t *rec = lds + (b * ng + g) * REC;
#pragma unroll
                    for (int gq = 0; gq < 4; gq++) {
                        const int j = 8 * hh + 2 * gq + t;
                        const int isum = dot16(q[gq], *(const int4 *)(rec + 16 * j), 0);
                        const int bs = (int)*(const int16_t *)(rec + REC_BSUMS + 2 * j);
                        // sum (q6 - 32) * x = sum q6 * x - 32 * (sum of the same 16 x)
                        S[b] += byte_s(scw[j >> 2], j & 3) * (isum - 32 * bs);
                    }
                }
            }
        }
    }
    const float dw = f16_bits_to_f32(W.d);
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const float dx = *(const float *)(lds + (b * ng + g) * REC + REC_D);
            f[b] += (dw * dx) * (float)S[b];
            if (DUMP) {
                So[b] = S[b];
                Smo[b] = 0;
            }
        }
    }
}

// ------------------------------------------------------------- Q2_K, Q3_K
// Both: element 128hf + 32j + 16t + i (half hf, shift j, 16-element half t)
// is bits 2j..2j+1 of qs byte 32hf + 16t + i, in 16-element group
// 8hf + 2j + t.  Q2_K: pieces 0 = scales (scale | min << 4 per group),
// 1 + 2hf + t = qs.  Q3_K: pieces t = hmask bytes 16t.., 2 + 2hf + t = qs,
// 6 = scales[12] then d; bit 4hf + j of the hmask byte set means the value
// is the two bits, clear means the two bits - 4, and the 6-bit group scale
// (candle's auxs form) is used as scale - 32.
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q2k(const Wt<TYPE_Q2_K> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], int (&So)[B], int (&Smo)[B]) {
    const uint32_t scw[4] = {W.pc[0].x, W.pc[0].y, W.pc[0].z, W.pc[0].w};
    int S[B];
#pragma unroll
    for (int b = 0; b < B; b++) S[b] = 0;
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint4 Q = W.pc[1 + 2 * hf + t];
            const uint32_t qv[4] = {Q.x, Q.y, Q.z, Q.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t q[4];
#pragma unroll
                for (int i = 0; i < 4; i++) q[i] = (qv[i] >> (2 * j)) & 0x03030303u;
                const int grp = 8 * hf + 2 * j + t;
                const int sc = byte_u(scw[grp >> 2], grp & 3) & 15;
#pragma unroll
                for (int b = 0; b < B; b++) {
                    if (b < m) {
                        const uint8_t *rec = lds + (b * ng + g) * REC;
                        S[b] += sc * dot16(q, *(const int4 *)(rec + 128 * hf + 32 * j + 16 * t), 0);
                    }
                }
            }
        }
    }
    const float dw = f16_bits_to_f32(W.d), dmw = f16_bits_to_f32(W.d >> 16);
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const uint8_t *rec = lds + (b * ng + g) * REC;
            const int4 p0 = *(const int4 *)(rec + REC_BSUMS), p1 = *(const int4 *)(rec + REC_BSUMS + 16);
            const uint32_t pw[8] = {(uint32_t)p0.x, (uint32_t)p0.y, (uint32_t)p0.z, (uint32_t)p0.w,
                                    (uint32_t)p1.x, (uint32_t)p1.y, (uint32_t)p1.z, (uint32_t)p1.w};
            int smin = 0;
#pragma unroll
            for (int w = 0; w < 8; w++) {  // bsums dword w: groups 2w, 2w + 1
                smin += (byte_u(scw[w >> 1], 2 * (w & 1)) >> 4) * lo16(pw[w]);
                smin += (byte_u(scw[w >> 1], 2 * (w & 1) + 1) >> 4) * hi16(pw[w]);
            }
            const float dx = *(const float *)(rec + REC_D);
            f[b] += (dw * dx) * (float)S[b] - (dmw * dx) * (float)smin;
            if (DUMP) {
                So[b] = S[b];
                Smo[b] = smin;
            }
        }
    }
}

template <int B, bool DUMP>
__device__ __forceinline__ void dot_q3k(const Wt<TYPE_Q3_K> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], int (&So)[B], int (&Smo)[B]) {
    const uint32_t a0 = W.pc[6].x, a1 = W.pc[6].y, tmp = W.pc[6].z;
    const uint32_t scw[4] = {(a0 & 0x0F0F0F0Fu) | ((tmp & 0x03030303u) << 4),
                             (a1 & 0x0F0F0F0Fu) | (((tmp >> 2) & 0x03030303u) << 4),
                             ((a0 >> 4) & 0x0F0F0F0Fu) | (((tmp >> 4) & 0x03030303u) << 4),
                             ((a1 >> 4) & 0x0F0F0F0Fu) | (((tmp >> 6) & 0x03030303u) << 4)};
    int S[B];
#pragma unroll
    for (int b = 0; b < B; b++) S[b] = 0;
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint4 Q = W.pc[2 + 2 * hf + t], H = W.pc[t];
            const uint32_t qv[4] = {Q.x, Q.y, Q.z, Q.w}, hv[4] = {H.x, H.y, H.z, H.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t q[4];  // value + 4, in 0..7
#pragma unroll
                for (int i = 0; i < 4; i++)
                    q[i] = ((qv[i] >> (2 * j)) & 0x03030303u) | (((hv[i] >> (4 * hf + j)) & 0x01010101u) << 2);
                const int grp = 8 * hf + 2 * j + t;
                const int sc = byte_u(scw[grp >> 2], grp & 3) - 32;
#pragma unroll
                for (int b = 0; b < B; b++) {
                    if (b < m) {
                        const uint8_t *rec = lds + (b * ng + g) * REC;
                        const int isum = dot16(q, *(const int4 *)(rec + 128 * hf + 32 * j + 16 * t), 0);
                        const int bs = (int)*(const int16_t *)(rec + REC_BSUMS + 2 * grp);
                        // sum (u - 4) * x = sum u * x - 4 * (sum of the same 16 x)
                        S[b] += sc * (isum - 4 * bs);
                    }
                }
            }
        }
    }
    const float dw = f16_bits_to_f32(W.pc[6].w);
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const float dx = *(const float *)(lds + (b * ng + g) * REC + REC_D);
            f[b] += (dw * dx) * (float)S[b];
            if (DUMP) {
                So[b] = S[b];
                Smo[b] = 0;
            }
        }
    }
}

// ------------------------------------------------------------------ Q8_0
// Group of eight blocks: pieces 2j, 2j+1 = qs of block j, piece 16 = the
// eight f16 d.  candle: sumf += (sum_i qw*qx as f32) * f16(d_w) * f16(d_x).
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q80(const Wt<TYPE_Q8_0> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], const MvParams &p, int row, bool row_ok) {
    const uint32_t dwp[4] = {W.pc[16].x, W.pc[16].y, W.pc[16].z, W.pc[16].w};
    const int nblk = p.k / QK8_0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint4 q0 = W.pc[2 * j], q1 = W.pc[2 * j + 1];
        const uint32_t qa[4] = {q0.x, q0.y, q0.z, q0.w}, qb[4] = {q1.x, q1.y, q1.z, q1.w};
        const float dw = f16_bits_to_f32(dwp[j >> 1] >> (16 * (j & 1)));
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (b < m) {
                const uint8_t *rec = lds + (b * ng + g) * REC;
                int isum = dot16(qa, *(const int4 *)(rec + 32 * j), 0);
                isum = dot16(qb, *(const int4 *)(rec + 32 * j + 16), isum);
                const float dx = *(const float *)(rec + REC_D8 + 4 * j);
                f[b] += ((float)isum * dw) * dx;
                if (DUMP) {
                    const int blk = 8 * g + j;
                    if (blk < nblk && row_ok) {
                        const int64_t o = ((int64_t)b * p.n + row) * nblk + blk;
                        p.S[o] = isum;
                        p.Smin[o] = 0;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------ Q4_0
// Group of eight blocks: piece j = the 16 qs bytes of block j (low nibbles
// elements 0..15, high nibbles 16..31, value q - 8), piece 8 = the eight f16
// d.  candle: sum_i ((q - 8) * qx) as f32 * f16(d_w) * f16(d_x); the integer
// sum is formed as sum q*qx - 8 * sum qx.
template <int B, bool DUMP>
__device__ __forceinline__ void dot_q40(const Wt<TYPE_Q4_0> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], const MvParams &p, int row, bool row_ok) {
    const uint32_t dwp[4] = {W.pc[8].x, W.pc[8].y, W.pc[8].z, W.pc[8].w};
    const uint32_t ones[4] = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
    const int nblk = p.k / QK8_0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint4 q = W.pc[j];
        const uint32_t lo[4] = {q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu};
        const uint32_t hi[4] = {(q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                                (q.w >> 4) & 0x0F0F0F0Fu};
        const float dw = f16_bits_to_f32(dwp[j >> 1] >> (16 * (j & 1)));
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (b < m) {
                const uint8_t *rec = lds + (b * ng + g) * REC;
                const int4 x0 = *(const int4 *)(rec + 32 * j), x1 = *(const int4 *)(rec + 32 * j + 16);
                int isum = dot16(lo, x0, 0);
                isum = dot16(hi, x1, isum);
                int xs = dot16(ones, x0, 0);
                xs = dot16(ones, x1, xs);
                isum -= 8 * xs;
                const float dx = *(const float *)(rec + REC_D8 + 4 * j);
                f[b] += ((float)isum * dw) * dx;
                if (DUMP) {
                    const int blk = 8 * g + j;
                    if (blk < nblk && row_ok) {
                        const int64_t o = ((int64_t)b * p.n + row) * nblk + blk;
                        p.S[o] = isum;
                        p.Smin[o] = 0;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------ Q5_0
// Group of eight blocks: piece j = the 16 qs bytes of block j, pieces 8, 9 =
// the 32-bit qh of blocks 0..3, 4..7, piece 10 = the eight f16 d.  Element
// e < 16: (qs[e] & 15) | bit e of qh << 4; element 16 + e: (qs[e] >> 4) |
// bit 16 + e of qh << 4; value - 16 (GGML dequantize_row_q5_0).  candle:
// sum_i (x * qx) as f32 * f16(d_w) * f16(d_x), the integer sum formed as
// sum q*qx - 16 * sum qx.  Four qh bits go to bit 4 of four bytes with one
// 24-bit multiply (spread4).

template <int B, bool DUMP>
__device__ __forceinline__ void dot_q50(const Wt<TYPE_Q5_0> &W, const uint8_t *lds, int ng, int g, int m,
                                        float (&f)[B], const MvParams &p, int row, bool row_ok) {
    const uint32_t dwp[4] = {W.pc[10].x, W.pc[10].y, W.pc[10].z, W.pc[10].w};
    const uint32_t qhw[8] = {W.pc[8].x, W.pc[8].y, W.pc[8].z, W.pc[8].w, W.pc[9].x, W.pc[9].y, W.pc[9].z, W.pc[9].w};
    const uint32_t ones[4] = {0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
    const int nblk = p.k / QK8_0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint4 q = W.pc[j];
        const uint32_t qv[4] = {q.x, q.y, q.z, q.w};
        const uint32_t h = qhw[j];
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = (qv[i] & 0x0F0F0F0Fu) | spread4((h >> (4 * i)) & 0xFu);
            hi[i] = ((qv[i] >> 4) & 0x0F0F0F0Fu) | spread4((h >> (16 + 4 * i)) & 0xFu);
        }
        const float dw = f16_bits_to_f32(dwp[j >> 1] >> (16 * (j & 1)));
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (b < m) {
                const uint8_t *rec = lds + (b * ng + g) * REC;
                const int4 x0 = *(const int4 *)(rec + 32 * j), x1 = *(const int4 *)(rec + 32 * j + 16);
                int isum = dot16(lo, x0, 0);
                isum = dot16(hi, x1, isum);
                int xs = dot16(ones, x0, 0);
                xs = dot16(ones, x1, xs);
                isum -= 16 * xs;
                const float dx = *(const float *)(rec + REC_D8 + 4 * j);
                f[b] += ((float)isum * dw) * dx;
                if (DUMP) {
                    const int blk = 8 * g + j;
                    if (blk < nblk && row_ok) {
                        const int64_t o = ((int64_t)b * p.n + row) * nblk + blk;
                        p.S[o] = isum;
                        p.Smin[o] = 0;
                    }
                }
            }
        }
    }
}

template <int TYPE, int B, bool DUMP>
__device__ __forceinline__ void group_dot(const Wt<TYPE> &W, const uint8_t *lds, const MvParams &p, int g, int row,
                                          bool valid, float (&f)[B]) {
    if (TYPE == TYPE_Q8_0) {
        dot_q80<B, DUMP>(*(const Wt<TYPE_Q8_0> *)&W, lds, p.ng, g, p.m, f, p, row, valid);
    } else if (TYPE == TYPE_Q4_0) {
        dot_q40<B, DUMP>(*(const Wt<TYPE_Q4_0> *)&W, lds, p.ng, g, p.m, f, p, row, valid);
    } else if (TYPE == TYPE_Q5_0) {
        dot_q50<B, DUMP>(*(const Wt<TYPE_Q5_0> *)&W, lds, p.ng, g, p.m, f, p, row, valid);
    } else {
        int So[B], Smo[B];
        if (TYPE == TYPE_Q4_K) dot_q45k<B, DUMP, TYPE_Q4_K>(*(const Wt<TYPE_Q4_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        else if (TYPE == TYPE_Q5_K) dot_q45k<B, DUMP, TYPE_Q5_K>(*(const Wt<TYPE_Q5_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        else if (TYPE == TYPE_Q2_K) dot_q2k<B, DUMP>(*(const Wt<TYPE_Q2_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        else if (TYPE == TYPE_Q3_K) dot_q3k<B, DUMP>(*(const Wt<TYPE_Q3_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        else dot_q6k<B, DUMP>(*(const Wt<TYPE_Q6_K> *)&W, lds, p.ng, g, p.m, f, So, Smo);
        if (DUMP && valid) {
#pragma unroll
            for (int b = 0; b < B; b++) {
                if (b < p.m) {
                    const int64_t o = ((int64_t)b * p.n + row) * p.ng + g;
                    p.S[o] = So[b];
                    p.Smin[o] = Smo[b];
                }
            }
        }
    }
}

// Activation of this pass into LDS records.  The global loads of the first
// PRE records of each wave (rec_load) are issued before the weight loads of
// the first iteration, so quantising them (rec_store) waits only for them.
constexpr int NW = 8;    // wavefronts per workgroup, at most
constexpr int PRE = 4;   // records per wave whose loads precede the weight loads

constexpr int XF_NONE = 0, XF_NORM = 1, XF_SILU = 2;

struct ActStage {
    u32x4 q[PRE];   // f32 inputs (fused) or quant bytes / bsums (pre-quantised)
    u32x4 q2[PRE];  // XF_NORM: the residual delta; XF_SILU: u
    u32x4 q3[PRE];  // XF_NORM: the norm weight
    float dsc[PRE];
};

// Record t = (batch row b, group g) of this pass.  Every lane issues the same
// loads whatever t is (records past the end read zeros).
template <int TYPE, bool FUSED, int XF = XF_NONE>
__device__ __forceinline__ void rec_load(ActStage &st, int r, const MvParams &p, int t, int lane) {
    const int ng = p.ng, k = p.k, m = p.m;
    const bool ok = t < m * ng;
    const int b = t / ng, g = t - b * ng;
    if (FUSED) {
        const rsrc_t rx = buf_rsrc(p.x, (uint32_t)(m * k * 4));
        uint32_t off;
        if (!act_q80(TYPE)) {
            off = ok ? (uint32_t)((b * k + g * QK_K + 4 * lane) * 4) : BUF_OOB;
        } else {
            const int j = lane >> 3, sub = lane & 7;
            off = ok && (8 * g + j) * QK8_0 < k ? (uint32_t)((b * k + (8 * g + j) * QK8_0 + 4 * sub) * 4) : BUF_OOB;
        }
        st.q[r] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
        if (XF == XF_NORM) {  // m = 1: the same offsets address delta and the norm weight
            const rsrc_t rdl = buf_rsrc(p.xdelta, p.xdelta ? (uint32_t)(k * 4) : 0u);
            const rsrc_t rnw = buf_rsrc(p.xnorm, (uint32_t)(k * 4));
            st.q2[r] = __builtin_amdgcn_raw_buffer_load_b128(rdl, off, 0, 0);
            st.q3[r] = __builtin_amdgcn_raw_buffer_load_b128(rnw, off, 0, 0);
        } else if (XF == XF_SILU) {
            const rsrc_t ru = buf_rsrc(p.x + k, (uint32_t)(k * 4));
            st.q2[r] = __builtin_amdgcn_raw_buffer_load_b128(ru, off, 0, 0);
        }
    } else if (!act_q80(TYPE)) {
        const rsrc_t rq = buf_rsrc(p.act.qs, (uint32_t)(m * k));
        const rsrc_t rs = buf_rsrc(p.act.bsums, (uint32_t)(m * (k / 16) * 2));
        const rsrc_t rd = buf_rsrc(p.act.d, (uint32_t)(m * (k / QK_K) * 4));
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rq, ok && lane < 16 ? (uint32_t)(b * k + g * QK_K + 16 * lane) : BUF_OOB, 0, 0);
        const u32x4 bs = __builtin_amdgcn_raw_buffer_load_b128(
            rs, ok && (unsigned)(lane - 16) < 2u ? (uint32_t)((b * (k / 16) + g * 16 + 8 * (lane - 16)) * 2) : BUF_OOB, 0, 0);
        const uint32_t d = __builtin_amdgcn_raw_buffer_load_b32(rd, ok && lane == 18 ? (uint32_t)((b * (k / QK_K) + g) * 4) : BUF_OOB, 0, 0);
        st.q[r] = lane < 16 ? q : bs;
        st.dsc[r] = u32_as_f32(d);
    } else {
        const int nblk = k / QK8_0;
        const rsrc_t rq = buf_rsrc(p.act.qs, (uint32_t)(m * k));
        const rsrc_t rd = buf_rsrc(p.act.d, (uint32_t)(m * nblk * 4));
        const int jq = lane >> 1, jd = lane - 16;
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(
            rq, ok && lane < 16 && 8 * g + jq < nblk ? (uint32_t)(b * k + (8 * g + jq) * QK8_0 + 16 * (lane & 1)) : BUF_OOB, 0, 0);
        const uint32_t d = __builtin_amdgcn_raw_buffer_load_b32(
            rd, ok && (unsigned)jd < 8u && 8 * g + jd < nblk ? (uint32_t)((b * nblk + 8 * g + jd) * 4) : BUF_OOB, 0, 0);
        st.q[r] = q;
        st.dsc[r] = u32_as_f32(d);
    }
}

template <int TYPE, bool FUSED>
__device__ __forceinline__ void rec_store(const ActStage &st, int r, uint8_t *lds, int t, int lane) {
    uint8_t *rec = lds + t * REC;
    if (FUSED) {
        const u32x4 u = st.q[r];
        const float v[4] = {u32_as_f32(u.x), u32_as_f32(u.y), u32_as_f32(u.z), u32_as_f32(u.w)};
        if (!act_q80(TYPE)) {
            int bsum;
            float d;
            const uint32_t packed = q8k_block_wave(v, lane, &bsum, &d);
            *(uint32_t *)(rec + 4 * lane) = packed;
            if ((lane & 3) == 0) *(int16_t *)(rec + REC_BSUMS + 2 * (lane >> 2)) = (int16_t)bsum;
            if (lane == 0) *(float *)(rec + REC_D) = d;
        } else {
            const int j = lane >> 3, sub = lane & 7;
            uint16_t h;
            const uint32_t packed = q8_0_block_8lanes(v, &h);  // a padding block is all zeros: q = 0, d = 0
            *(uint32_t *)(rec + 32 * j + 4 * sub) = packed;
            if (sub == 0) *(float *)(rec + REC_D8 + 4 * j) = f16_bits_to_f32(h);
        }
    } else {
        if (!act_q80(TYPE)) {
            if (lane < 16) *(u32x4 *)(rec + 16 * lane) = st.q[r];
            else if (lane < 18) *(u32x4 *)(rec + REC_BSUMS + 16 * (lane - 16)) = st.q[r];
            else if (lane == 18) *(float *)(rec + REC_D) = st.dsc[r];
        } else {
            if (lane < 16) *(u32x4 *)(rec + 16 * lane) = st.q[r];
            else if (lane < 24) *(float *)(rec + REC_D8 + 4 * (lane - 16)) = st.dsc[r];
        }
    }
}

// silu(g) * u of four elements (candle: x / (1 + e^-x)).
__device__ __forceinline__ u32x4 silu_mul4(u32x4 g, u32x4 u) {
    const float gv[4] = {u32_as_f32(g.x), u32_as_f32(g.y), u32_as_f32(g.z), u32_as_f32(g.w)};
    const float uv[4] = {u32_as_f32(u.x), u32_as_f32(u.y), u32_as_f32(u.z), u32_as_f32(u.w)};
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = (gv[i] / (1.0f + expf(-gv[i]))) * uv[i];
    return (u32x4){f32_as_u32(o[0]), f32_as_u32(o[1]), f32_as_u32(o[2]), f32_as_u32(o[3])};
}

// The matvec of one workgroup (bid of nblk): the kernel body, shared by
// matvec_kernel and by matvec2_kernel, which runs two weights' matvecs on the
// same input in one launch.
template <int TYPE, int B, bool DUMP, bool FUSED, int XF>
__device__ __forceinline__ void matvec_body(const MvParams &p, const int bid, const int nblk, uint8_t *lds) {
    static_assert(XF == XF_NONE || (FUSED && B == 1), "input transforms are for one f32 row");
    __shared__ float red[NW][B][RB];  // per-wavefront chunk partials of the 8 rows of a row block
    __shared__ float nred[NW];        // XF_NORM: per-wavefront sums of squares
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int g_l = lane >> 3, r_l = lane & 7;
    const int nw = p.nw, nsub = p.nsub;
    const int np = p.np;                     // wavefronts (chunk partials) per row block
    const int rbo = wave / np;               // row block of this wavefront within an iteration
    const int c0 = wave - rbo * np;          // its first chunk; step j takes chunk c0 + np * j
    const int nrb = (p.n + RB - 1) / RB;
    const int nrec = p.m * p.ng;
    const int nsteps = p.iters * nsub;
    // a step past the last reads zeros: blockIdx + iters * gridDim >= workgroup iterations
    auto rb_of = [&](int st) { return (int)(bid + (st / nsub) * nblk) * p.rbw + rbo; };
    auto g_of = [&](int st) { return 8 * (c0 + np * (st % nsub)) + g_l; };

    // 1. activation loads of the first records, 2. weight loads of the first
    // step, 3. quantise / copy into LDS (waits only for step 1).
    ActStage as;
#pragma unroll
    for (int r = 0; r < PRE; r++) rec_load<TYPE, FUSED, XF>(as, r, p, wave + nw * r, lane);
    Wt<TYPE> wa, wb;
    load_w<TYPE>(wa, p, rb_of(0), nrb, g_of(0), r_l);
    if (XF == XF_NORM) {
        // every record of the row is among the first PRE per wavefront (the
        // launcher checks), so the row's sum of squares is known before any
        // record is quantised; records past the end loaded zeros
        float ss = 0.0f;
#pragma unroll
        for (int r = 0; r < PRE; r++) {
            const u32x4 x4 = as.q[r], d4 = as.q2[r];
            const float h[4] = {u32_as_f32(x4.x) + u32_as_f32(d4.x), u32_as_f32(x4.y) + u32_as_f32(d4.y),
                                u32_as_f32(x4.z) + u32_as_f32(d4.z), u32_as_f32(x4.w) + u32_as_f32(d4.w)};
            as.q[r] = (u32x4){f32_as_u32(h[0]), f32_as_u32(h[1]), f32_as_u32(h[2]), f32_as_u32(h[3])};
#pragma unroll
            for (int i = 0; i < 4; i++) ss = __builtin_fmaf(h[i], h[i], ss);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
        if (lane == 0) nred[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int w = 0; w < nw; w++) tot += nred[w];
        const float mden = sqrtf(tot / (float)p.k + p.eps);
        const float rm = 1.0f / mden;  // candle's h / m as h * (1 / m), as the row-per-lane kernel forms it
        const rsrc_t rxo = buf_rsrc(p.xout, p.xout && bid == 0 ? (uint32_t)(p.k * 4) : 0u);
#pragma unroll
        for (int r = 0; r < PRE; r++) {
            const int t = wave + nw * r;
            uint32_t off = BUF_OOB;
            if (!act_q80(TYPE)) {
                if (t < nrec) off = (uint32_t)((t * QK_K + 4 * lane) * 4);
            } else {
                const int j = lane >> 3, sub = lane & 7;
                if (t < nrec && (8 * t + j) * QK8_0 < p.k) off = (uint32_t)(((8 * t + j) * QK8_0 + 4 * sub) * 4);
            }
            __builtin_amdgcn_raw_buffer_store_b128(as.q[r], rxo, off, 0, 0);  // the residual stream x + delta
            const u32x4 h4 = as.q[r], w4 = as.q3[r];
            as.q[r] = (u32x4){f32_as_u32((u32_as_f32(h4.x) * rm) * u32_as_f32(w4.x)),
                              f32_as_u32((u32_as_f32(h4.y) * rm) * u32_as_f32(w4.y)),
                              f32_as_u32((u32_as_f32(h4.z) * rm) * u32_as_f32(w4.z)),
                              f32_as_u32((u32_as_f32(h4.w) * rm) * u32_as_f32(w4.w))};
        }
    } else if (XF == XF_SILU) {
#pragma unroll
        for (int r = 0; r < PRE; r++) as.q[r] = silu_mul4(as.q[r], as.q2[r]);
    }
#pragma unroll
    for (int r = 0; r < PRE; r++) {
        const int t = wave + nw * r;
        if (t < nrec) rec_store<TYPE, FUSED>(as, r, lds, t, lane);
    }
    for (int t = wave + nw * PRE; t < nrec; t += nw) {  // none with XF_NORM
        rec_load<TYPE, FUSED, XF>(as, 0, p, t, lane);
        if (XF == XF_SILU) as.q[0] = silu_mul4(as.q[0], as.q2[0]);
        rec_store<TYPE, FUSED>(as, 0, lds, t, lane);
    }
    __syncthreads();

    float f[B];
#pragma unroll
    for (int b = 0; b < B; b++) f[b] = 0.0f;
    const rsrc_t ry = buf_rsrc(p.y, (uint32_t)(p.m * p.n * 4));

    // Row block partials of iteration it: butterfly over the chunk's 8 groups
    // of each row (lanes r_l, r_l + 8, ..., r_l + 56); with several wavefronts
    // per row block, lane r of wavefront w < rbw then sums row r of row block
    // w's partials in chunk order (the other lanes' stores are dropped).
    auto finish = [&](int it) {
#pragma unroll
        for (int b = 0; b < B; b++) {
            f[b] += __shfl_xor(f[b], 8);
            f[b] += __shfl_xor(f[b], 16);
            f[b] += __shfl_xor(f[b], 32);
        }
        if (np == 1) {  // workgroup-uniform: this wavefront holds whole rows, lanes 0..7 store them
            const int row = rb_of(it * nsub) * RB + r_l;
            const bool ok = lane < RB && row < p.n;
#pragma unroll
            for (int b = 0; b < B; b++) {
                __builtin_amdgcn_raw_buffer_store_b32(f32_as_u32(f[b]), ry,
                                                      ok && b < p.m ? (uint32_t)((b * p.n + row) * 4) : BUF_OOB, 0, 0);
                f[b] = 0.0f;
            }
            return;
        }
        if (g_l == 0) {
#pragma unroll
            for (int b = 0; b < B; b++) red[wave][b][r_l] = f[b];
        }
#pragma unroll
        for (int b = 0; b < B; b++) f[b] = 0.0f;
        __syncthreads();
        const int wr = wave < p.rbw ? wave : 0;
        const int row = ((int)(bid + it * nblk) * p.rbw + wr) * RB + r_l;
        const bool ok = wave < p.rbw && lane < RB && row < p.n;
#pragma unroll
        for (int b = 0; b < B; b++) {
            float s = 0.0f;
            for (int c = 0; c < np; c++) s += red[wr * np + c][b][r_l];
            __builtin_amdgcn_raw_buffer_store_b32(f32_as_u32(s), ry,
                                                  ok && b < p.m ? (uint32_t)((b * p.n + row) * 4) : BUF_OOB, 0, 0);
        }
        __syncthreads();
    };
    // No branch around the dot product: a row block past the end holds zero
    // weights (its loads read zeros), which add nothing, and keeping every
    // path alike keeps the compiler's s_waitcnt counts exact.
    auto step = [&](const Wt<TYPE> &W, int st) {
        const int g = g_of(st), row = rb_of(st) * RB + r_l;
        group_dot<TYPE, B, DUMP>(W, lds, p, g < p.ng ? g : p.ng - 1, row, row < p.n && g < p.ng, f);
        if (st % nsub == nsub - 1) finish(st / nsub);  // workgroup-uniform
    };

    // ping-pong: wa holds step st, wb step st + 1
    for (int st = 0; st < nsteps; st += 2) {
        load_w<TYPE>(wb, p, rb_of(st + 1), nrb, g_of(st + 1), r_l);
        step(wa, st);
        if (st + 1 >= nsteps) break;
        load_w<TYPE>(wa, p, rb_of(st + 2), nrb, g_of(st + 2), r_l);
        step(wb, st + 1);
    }
}

template <int TYPE, int B, bool DUMP, bool FUSED, int XF = XF_NONE>
__global__ __launch_bounds__(NW * 64) void matvec_kernel(MvParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    matvec_body<TYPE, B, DUMP, FUSED, XF>(p, (int)blockIdx.x, (int)gridDim.x, lds);
}

// Two matvecs of one f32 row (m = 1) in one launch: workgroups below grid1
// run weight 1 (type T1, p1), the rest weight 2 (T2, p2).  Both plans use
// NW wavefronts per workgroup; the dynamic LDS is the larger of the two.
template <int T1, int T2, int XF>
__global__ __launch_bounds__(NW * 64) void matvec2_kernel(MvParams p1, MvParams p2, int grid1) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int bid = (int)blockIdx.x;
    if (bid < grid1) matvec_body<T1, 1, false, true, XF>(p1, bid, grid1, lds);  // uniform over the workgroup
    else matvec_body<T2, 1, false, true, XF>(p2, bid - grid1, (int)gridDim.x - grid1, lds);
}

// Dynamic LDS above 64 KB has to be allowed per kernel, once.
template <int TYPE, int B>
hipError_t allow_lds() {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        const int cap = (int)LDS_CAP;
        const void *fns[4] = {(const void *)matvec_kernel<TYPE, B, false, false>,
                              (const void *)matvec_kernel<TYPE, B, false, true>,
                              (const void *)matvec_kernel<TYPE, B, true, false>,
                              (const void *)matvec_kernel<TYPE, B, true, true>};
        for (const void *f : fns) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, cap);
            if (e != hipSuccess) err = e;
        }
    });
    return err;
}

template <int TYPE>
hipError_t allow_lds_xf() {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        const int cap = (int)LDS_CAP;
        const void *fns[2] = {(const void *)matvec_kernel<TYPE, 1, false, true, XF_NORM>,
                              (const void *)matvec_kernel<TYPE, 1, false, true, XF_SILU>};
        for (const void *f : fns) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, cap);
            if (e != hipSuccess) err = e;
        }
    });
    return err;
}

template <int TYPE, int B>
hipError_t launch_tb(const MvParams &p, unsigned grid, size_t lds, bool dump, int xf, hipStream_t s) {
    const dim3 blk(p.nw * 64);
    if (xf != XF_NONE) {
        if (B != 1 || dump || !p.x) return hipErrorInvalidValue;
        if (lds > 64 * 1024) {
            const hipError_t e = allow_lds_xf<TYPE>();
            if (e != hipSuccess) return e;
        }
        if (xf == XF_NORM) matvec_kernel<TYPE, 1, false, true, XF_NORM><<<grid, blk, lds, s>>>(p);
        else matvec_kernel<TYPE, 1, false, true, XF_SILU><<<grid, blk, lds, s>>>(p);
        return hipGetLastError();
    }
    if (lds > 64 * 1024) {
        const hipError_t e = allow_lds<TYPE, B>();
        if (e != hipSuccess) return e;
    }
    if (p.x) {
        if (dump) matvec_kernel<TYPE, B, true, true><<<grid, blk, lds, s>>>(p);
        else matvec_kernel<TYPE, B, false, true><<<grid, blk, lds, s>>>(p);
    } else {
        if (dump) matvec_kernel<TYPE, B, true, false><<<grid, blk, lds, s>>>(p);
        else matvec_kernel<TYPE, B, false, false><<<grid, blk, lds, s>>>(p);
    }
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_t(int B, const MvParams &p, unsigned grid, size_t lds, bool dump, int xf, hipStream_t s) {
    switch (B) {
    case 1: return launch_tb<TYPE, 1>(p, grid, lds, dump, xf, s);
    case 2: return launch_tb<TYPE, 2>(p, grid, lds, dump, xf, s);
    case 4: return launch_tb<TYPE, 4>(p, grid, lds, dump, xf, s);
    case 8: return launch_tb<TYPE, 8>(p, grid, lds, dump, xf, s);
    default: return hipErrorInvalidConfiguration;
    }
}

struct XfArgs {
    int xf = XF_NONE;
    const float *delta = nullptr, *norm = nullptr;
    float eps = 0.0f;
    float *xout = nullptr;
};

// Launch shape of a matvec over n rows of ng groups.
struct MvPlan {
    int nch, np, rbw, nw, nsub;
    int64_t iters, grid;
};
MvPlan mv_plan(int64_t n, int ng) {
    MvPlan P;
    const int64_t nrb = (n + RB - 1) / RB;
    // Wavefronts per row block: as few as give MIN_WAVES wavefronts in all
    // (fewer, longer-lived wavefronts keep two steps of loads in flight and
    // need no cross-wavefront reduction), at most one per chunk and NW.
    P.nch = (ng + 7) / 8;  // 8-group chunks per row
    P.np = 1;
    while (P.np < NW && P.np < P.nch && nrb * P.np < MIN_WAVES) P.np *= 2;
    if (P.np > P.nch) P.np = P.nch;
    P.rbw = NW / P.np;                        // row blocks per workgroup iteration
    P.nw = P.rbw * P.np;                      // wavefronts per workgroup
    P.nsub = (P.nch + P.np - 1) / P.np;       // chunks per wavefront per row block
    const int64_t wg_iters = (nrb + P.rbw - 1) / P.rbw;  // workgroup iterations in total
    const int64_t target_wg = TARGET_WAVES / P.nw;
    P.iters = (wg_iters + target_wg - 1) / target_wg;
    P.grid = (wg_iters + P.iters - 1) / P.iters;
    return P;
}

hipError_t matvec_impl(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act, int64_t m,
                       float *y, int32_t *S, int32_t *Smin, const XfArgs &xa, hipStream_t s);

hipError_t matvec_impl(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act, int64_t m,
                       float *y, int32_t *S, int32_t *Smin, const XfArgs &xa, hipStream_t s) {
    const int type = w.type;
    if (type != TYPE_Q4_K && type != TYPE_Q5_K && type != TYPE_Q6_K && type != TYPE_Q8_0 && type != TYPE_Q4_0 &&
        type != TYPE_Q2_K && type != TYPE_Q3_K && type != TYPE_Q5_0)
        return hipErrorInvalidValue;
    const int blk = act_q80(type) ? QK8_0 : QK_K;
    if (!w.slab || m < 0 || n <= 0 || k <= 0 || k % blk || n > 0x7fffffff || k > 0x7fffffff || !y)
        return hipErrorInvalidValue;
    if ((type == TYPE_Q6_K || type == TYPE_Q2_K) && !w.d) return hipErrorInvalidValue;
    if (w.ng != groups_of(type, k)) return hipErrorInvalidValue;
    if (!x && !act) return hipErrorInvalidValue;
    if (x && ((uintptr_t)x & 15)) return hipErrorInvalidValue;  // the fused prologue reads float4
    if ((S == nullptr) != (Smin == nullptr)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    if (xa.xf != XF_NONE && (m != 1 || !x || S || (xa.xf == XF_NORM && !xa.norm))) return hipErrorInvalidValue;
    if (m == 1 && xa.xf == XF_NONE && rowlane_matvec_applies(type, n, k)) {
        const hipError_t e = launch_rowlane_matvec(w, n, k, x, act, y, S, Smin, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (m == 1 && xa.xf != XF_NONE && rowlane_xf_applies(type, n, k, xa.xf == XF_NORM ? RL_XF_NORM : RL_XF_SILU)) {
        const RlXf rx{xa.xf == XF_NORM ? RL_XF_NORM : RL_XF_SILU, xa.delta, xa.norm, xa.eps, xa.xout};
        const hipError_t e = launch_rowlane_matvec(w, n, k, x, nullptr, y, nullptr, nullptr, s, &rx);
        if (e != hipErrorNotSupported) return e;
    }
    const int ng = w.ng;
    if ((size_t)ng * REC > LDS_CAP) return hipErrorNotSupported;  // k > 124160
    if ((int64_t)8 * n * 4 >= ((int64_t)1 << 31)) return hipErrorNotSupported;  // y of a pass: 32-bit buffer offsets
    const MvPlan P = mv_plan(n, ng);
    const int nch = P.nch, np = P.np, rbw = P.rbw, nw = P.nw, nsub = P.nsub;
    const int64_t iters = P.iters, grid = P.grid;
    if ((int64_t)iters * nsub > 0x7fffffff) return hipErrorInvalidValue;
    // the fused norm needs the whole row among each wavefront's first PRE records
    if (xa.xf == XF_NORM && ng > PRE * nw) return hipErrorNotSupported;
    const int64_t nblk = k / blk;
    int64_t r0 = 0;
    while (r0 < m) {
        const int64_t rem = m - r0;
        int B = rem >= 8 ? 8 : rem > 4 ? 8 : rem > 2 ? 4 : rem;
        while (B > 1 && (size_t)B * ng * REC > LDS_CAP) B >>= 1;
        const int mb = (int)(rem < B ? rem : B);
        MvParams p;
        p.w = w.slab;
        p.wd = w.d;
        p.rb_stride = w.rb_stride;
        p.n = (int)n;
        p.k = (int)k;
        p.ng = ng;
        p.nch = nch;
        p.np = np;
        p.rbw = rbw;
        p.nw = nw;
        p.nsub = nsub;
        p.m = mb;
        p.iters = (int)iters;
        p.x = x ? x + r0 * k : nullptr;
        p.xdelta = xa.delta;
        p.xnorm = xa.norm;
        p.xout = xa.xout;
        p.eps = xa.eps;
        if (act) {
            p.act.qs = act->qs + r0 * k;
            p.act.d = act->d + r0 * (k / blk);
            p.act.d16 = act->d16;
            p.act.bsums = act->bsums + r0 * (k / 16);
        } else {
            p.act = ActPlanes{};
        }
        p.y = y + r0 * n;
        p.S = S ? S + r0 * n * nblk : nullptr;
        p.Smin = Smin ? Smin + r0 * n * nblk : nullptr;
        const size_t lds = (size_t)B * ng * REC;
        hipError_t e;
        switch (type) {
        case TYPE_Q4_K: e = launch_t<TYPE_Q4_K>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        case TYPE_Q5_K: e = launch_t<TYPE_Q5_K>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        case TYPE_Q6_K: e = launch_t<TYPE_Q6_K>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        case TYPE_Q4_0: e = launch_t<TYPE_Q4_0>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        case TYPE_Q2_K: e = launch_t<TYPE_Q2_K>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        case TYPE_Q3_K: e = launch_t<TYPE_Q3_K>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        case TYPE_Q5_0: e = launch_t<TYPE_Q5_0>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        default: e = launch_t<TYPE_Q8_0>(B, p, (unsigned)grid, lds, S != nullptr, xa.xf, s); break;
        }
        if (e != hipSuccess) return e;
        r0 += mb;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_matvec(const WLayout &w, int64_t n, int64_t k, const float *x, const ActPlanes *act, int64_t m,
                         float *y, int32_t *S, int32_t *Smin, hipStream_t s) {
    return matvec_impl(w, n, k, x, act, m, y, S, Smin, XfArgs{}, s);
}

hipError_t launch_matvec_rmsnorm(const WLayout &w, int64_t n, int64_t k, const float *x, const float *delta,
                                 const float *norm, float eps, float *xout, float *y, hipStream_t s) {
    if ((delta && ((uintptr_t)delta & 15)) || !norm || ((uintptr_t)norm & 15) || (xout && ((uintptr_t)xout & 15)))
        return hipErrorInvalidValue;
    XfArgs xa;
    xa.xf = XF_NORM;
    xa.delta = delta;
    xa.norm = norm;
    xa.eps = eps;
    xa.xout = xout;
    return matvec_impl(w, n, k, x, nullptr, 1, y, nullptr, nullptr, xa, s);
}

hipError_t launch_matvec_rmsnorm_swiglu(const WLayout &w, int64_t n, int64_t k, const float *x, const float *delta,
                                        const float *norm, float eps, float *xout, float *h, hipStream_t s) {
    if ((delta && ((uintptr_t)delta & 15)) || !norm || ((uintptr_t)norm & 15) || (xout && ((uintptr_t)xout & 15)) ||
        n % 8)
        return hipErrorInvalidValue;
    if (!rowlane_xf_applies(w.type, n, k, RL_XF_NORM)) return hipErrorNotSupported;
    RlXf rx{RL_XF_NORM, delta, norm, eps, xout};
    rx.swiglu = true;
    return launch_rowlane_matvec(w, n, k, x, nullptr, h, nullptr, nullptr, s, &rx);
}

hipError_t launch_matvec_rmsnorm_argmax(const WLayout &w, int64_t n, int64_t k, const float *x, const float *delta,
                                        const float *norm, float eps, float *y, int2 *amax, int max_parts,
                                        int *nparts, hipStream_t s) {
    if ((delta && ((uintptr_t)delta & 15)) || !norm || ((uintptr_t)norm & 15) || !amax || !nparts)
        return hipErrorInvalidValue;
    if (!rowlane_xf_applies(w.type, n, k, RL_XF_NORM)) return hipErrorNotSupported;
    const int g = rowlane_grid(w.type, n, k);
    if (g <= 0 || g > max_parts) return hipErrorNotSupported;
    RlXf rx{RL_XF_NORM, delta, norm, eps, nullptr};
    rx.amax = amax;
    *nparts = g;
    return launch_rowlane_matvec(w, n, k, x, nullptr, y, nullptr, nullptr, s, &rx);
}

hipError_t launch_matvec_silu(const WLayout &w, int64_t n, int64_t k, const float *gu, float *y, hipStream_t s) {
    XfArgs xa;
    xa.xf = XF_SILU;
    return matvec_impl(w, n, k, gu, nullptr, 1, y, nullptr, nullptr, xa, s);
}

namespace {
// MvParams of a one-row fused-norm matvec, or an error.
hipError_t norm_params(const WLayout &w, int64_t n, int64_t k, const float *x, const XfArgs &xa, float *y,
                       MvParams &p, int64_t &grid, size_t &lds) {
    const int type = w.type;
    if (type != TYPE_Q4_K && type != TYPE_Q6_K && type != TYPE_Q5_0 && type != TYPE_Q8_0) return hipErrorNotSupported;
    const int blk = act_q80(type) ? QK8_0 : QK_K;
    if (!w.slab || n <= 0 || k <= 0 || k % blk || n > 0x7fffffff || k > 0x7fffffff || !y || !x) return hipErrorInvalidValue;
    if ((type == TYPE_Q6_K || type == TYPE_Q2_K) && !w.d) return hipErrorInvalidValue;
    if (w.ng != groups_of(type, k) || ((uintptr_t)x & 15) || !xa.norm) return hipErrorInvalidValue;
    const int ng = w.ng;
    if ((int64_t)8 * n * 4 >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    const MvPlan P = mv_plan(n, ng);
    if (ng > PRE * P.nw || P.nw != NW || P.iters * P.nsub > 0x7fffffff) return hipErrorNotSupported;
    p = MvParams{};
    p.w = w.slab;
    p.wd = w.d;
    p.rb_stride = w.rb_stride;
    p.n = (int)n;
    p.k = (int)k;
    p.ng = ng;
    p.nch = P.nch;
    p.np = P.np;
    p.rbw = P.rbw;
    p.nw = P.nw;
    p.nsub = P.nsub;
    p.m = 1;
    p.iters = (int)P.iters;
    p.x = x;
    p.xdelta = xa.delta;
    p.xnorm = xa.norm;
    p.xout = xa.xout;
    p.eps = xa.eps;
    p.y = y;
    grid = P.grid;
    lds = (size_t)ng * REC;
    return hipSuccess;
}

template <int T1, int T2>
hipError_t launch_two(const MvParams &p1, const MvParams &p2, int64_t g1, int64_t g2, size_t lds, hipStream_t s) {
    if (lds > 64 * 1024) {
        static std::once_flag once;
        static hipError_t err = hipSuccess;
        std::call_once(once, [] {
            err = hipFuncSetAttribute((const void *)matvec2_kernel<T1, T2, XF_NORM>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_CAP);
        });
        if (err != hipSuccess) return err;
    }
    matvec2_kernel<T1, T2, XF_NORM><<<(unsigned)(g1 + g2), NW * 64, lds, s>>>(p1, p2, (int)g1);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_matvec2_rmsnorm(const WLayout &w1, int64_t n1, float *y1, const WLayout &w2, int64_t n2, float *y2,
                                  int64_t k, const float *x, const float *delta, const float *norm, float eps,
                                  float *xout, hipStream_t s) {
    if ((delta && ((uintptr_t)delta & 15)) || !norm || ((uintptr_t)norm & 15) || (xout && ((uintptr_t)xout & 15)))
        return hipErrorInvalidValue;
    // The two weights' outputs equal their single calls' bytes: both
    // row-per-lane in one launch where the shapes allow, the general kernel
    // for both in one launch for the type pairs instantiated below (Q4_K /
    // Q6_K, and the Q5_0 / Q8_0 a Q4_K_M file holds for rows that are not
    // whole 256-element groups), one launch each otherwise.
    auto kq = [](int t) { return t == TYPE_Q4_K || t == TYPE_Q6_K; };
    auto q0 = [](int t) { return t == TYPE_Q5_0 || t == TYPE_Q8_0; };
    const bool pair_k = kq(w1.type) && kq(w2.type), pair_0 = q0(w1.type) && q0(w2.type);
    if (pair_k && (k % QK_K || k / QK_K > PRE * NW)) return hipErrorNotSupported;
    const bool r1 = rowlane_xf_applies(w1.type, n1, k, RL_XF_NORM), r2 = rowlane_xf_applies(w2.type, n2, k, RL_XF_NORM);
    if (r1 && r2 && pair_k) {
        const RlXf rx{RL_XF_NORM, delta, norm, eps, xout};
        const hipError_t e = launch_rowlane_matvec2(w1, n1, y1, w2, n2, y2, k, x, rx, s);
        if (e != hipErrorNotSupported) return e;
    }
    auto singles = [&]() {
        const hipError_t e = launch_matvec_rmsnorm(w1, n1, k, x, delta, norm, eps, xout, y1, s);
        if (e != hipSuccess) return e;
        return launch_matvec_rmsnorm(w2, n2, k, x, delta, norm, eps, nullptr, y2, s);
    };
    if (r1 || r2 || !(pair_k || pair_0)) return singles();
    XfArgs xa;
    xa.xf = XF_NORM;
    xa.delta = delta;
    xa.norm = norm;
    xa.eps = eps;
    xa.xout = xout;
    MvParams p1, p2;
    int64_t g1, g2;
    size_t l1, l2;
    hipError_t e = norm_params(w1, n1, k, x, xa, y1, p1, g1, l1);
    if (e == hipErrorNotSupported) return singles();
    if (e != hipSuccess) return e;
    xa.xout = nullptr;  // the residual is written once, by weight 1's workgroup 0
    if ((e = norm_params(w2, n2, k, x, xa, y2, p2, g2, l2)) == hipErrorNotSupported) return singles();
    if (e != hipSuccess) return e;
    if (g1 + g2 > 0x7fffffff) return singles();
    const size_t lds = l1 > l2 ? l1 : l2;
    const int t1 = w1.type, t2 = w2.type;
    if (pair_0) {
        if (t1 == TYPE_Q5_0 && t2 == TYPE_Q8_0) return launch_two<TYPE_Q5_0, TYPE_Q8_0>(p1, p2, g1, g2, lds, s);
        if (t1 == TYPE_Q5_0 && t2 == TYPE_Q5_0) return launch_two<TYPE_Q5_0, TYPE_Q5_0>(p1, p2, g1, g2, lds, s);
        if (t1 == TYPE_Q8_0 && t2 == TYPE_Q8_0) return launch_two<TYPE_Q8_0, TYPE_Q8_0>(p1, p2, g1, g2, lds, s);
        return launch_two<TYPE_Q8_0, TYPE_Q5_0>(p1, p2, g1, g2, lds, s);
    }
    if (t1 == TYPE_Q4_K && t2 == TYPE_Q6_K) return launch_two<TYPE_Q4_K, TYPE_Q6_K>(p1, p2, g1, g2, lds, s);
    if (t1 == TYPE_Q4_K && t2 == TYPE_Q4_K) return launch_two<TYPE_Q4_K, TYPE_Q4_K>(p1, p2, g1, g2, lds, s);
    if (t1 == TYPE_Q6_K && t2 == TYPE_Q4_K) return launch_two<TYPE_Q6_K, TYPE_Q4_K>(p1, p2, g1, g2, lds, s);
    return launch_two<TYPE_Q6_K, TYPE_Q6_K>(p1, p2, g1, g2, lds, s);
}

}  // namespace aq
