// k_crate.hip -- the NIF crate's own int8 / int4 kernels on gfx950
// (native/arm_ai_nif/src/shape_ops.rs; NIFs lib.rs:172-211, :213-296,
// :342-399, :401-532): int8 x int8 matmuls with per-tensor / per-token
// activation scales, the per-token int8 quantizer, weight-only matmuls with
// int8 / f16 / Q4_0-style int4 weights, the Q4_0 x Q8 GEMV, the Q4_0-style
// weight quantizer, and the row / tensor dequantizers.
//
// Exactness: integer dot products are exact and every per-element f32
// operation the crate performs on them (scalings, quantizer divisions and
// roundings) is the same IEEE operation here, so the int8 matmuls, the
// quantizers and the dequantizers are bit-identical to the crate's scalar
// code.  The f32 accumulations of the weight-only matmuls sum the same terms
// in a different order (a tree over lanes instead of a sequential loop).
#include "aq_internal.h"

namespace aq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int32_t sat_f2i(float v) {  // Rust `f as i32`
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// ---------------------------------------------------------------------------
// int8 x int8 -> f32, small m: one wavefront per (output column j, pass of
// up to 8 activation rows); lanes stride over K in 16-byte chunks
// (v_dot4_i32_i8), the tail byte by byte.  out = ((f32)acc * sa_i) * sw_j.
// ---------------------------------------------------------------------------
template <int B>
__global__ __launch_bounds__(256) void int8_rows_kernel(const int8_t *__restrict__ a, const int8_t *__restrict__ w,
                                                        const float *__restrict__ act_scales, float act_scale,
                                                        const float *__restrict__ w_scales, int m, int n, int64_t k,
                                                        float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= n) return;  // wave-uniform
    const int8_t *wr = w + j * k;
    int acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0;
    const int64_t k16 = k & ~(int64_t)15;
    for (int64_t c = (int64_t)lane * 16; c < k16; c += 64 * 16) {
        int wv[4];
        __builtin_memcpy(wv, wr + c, 16);
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (b < m) {
                int av[4];
                __builtin_memcpy(av, a + (int64_t)b * k + c, 16);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[b] = sdot4(av[i], wv[i], acc[b]);
            }
        }
    }
    for (int64_t c = k16 + lane; c < k; c += 64) {
#pragma unroll
        for (int b = 0; b < B; b++)
            if (b < m) acc[b] += (int)a[(int64_t)b * k + c] * (int)wr[c];
    }
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const int s = wave_sum(acc[b]);
            if (lane == 0) {
                const float sa = act_scales ? act_scales[b] : act_scale;
                out[(int64_t)b * n + j] = ((float)s * sa) * w_scales[j];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// int8 x int8 -> f32, larger m: one wavefront per 64 x 64 output block, four
// v_mfma_i32_32x32x32_i8 tiles; A and W fragments straight from global
// memory (L2-resident), the last partial K step masked to zero.
// MFMA operand layout: lane l holds K bytes 16*(l/32) .. +15 of row l%32;
// result element r of lane l is (row 8*(r/4) + 4*(l/32) + r%4, column l%32).
// ---------------------------------------------------------------------------
__device__ __forceinline__ v4i load16_masked(const int8_t *row, int64_t c, int64_t k) {
    v4i v = {0, 0, 0, 0};
    if (c + 16 <= k) {
        __builtin_memcpy(&v, row + c, 16);
    } else if (c < k) {
        int8_t t[16];
#pragma unroll
        for (int i = 0; i < 16; i++) t[i] = c + i < k ? row[c + i] : (int8_t)0;
        __builtin_memcpy(&v, t, 16);
    }
    return v;
}

__global__ __launch_bounds__(256) void int8_mfma_kernel(const int8_t *__restrict__ a, const int8_t *__restrict__ w,
                                                        const float *__restrict__ act_scales, float act_scale,
                                                        const float *__restrict__ w_scales, int m, int n, int64_t k,
                                                        float *__restrict__ out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    // workgroup: 128 x 128, wavefront (wave/2, wave%2): 64 x 64
    const int64_t m0 = (int64_t)blockIdx.y * 128 + (wave >> 1) * 64;
    const int64_t n0 = (int64_t)blockIdx.x * 128 + (wave & 1) * 64;
    if (m0 >= m || n0 >= n) return;  // wave-uniform; no barriers below
    const int8_t *ar[2], *wr[2];
    bool aok[2], wok[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int64_t r = m0 + 32 * t + l32, c = n0 + 32 * t + l32;
        aok[t] = r < m;
        wok[t] = c < n;
        ar[t] = a + (aok[t] ? r : 0) * k;
        wr[t] = w + (wok[t] ? c : 0) * k;
    }
    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int jx = 0; jx < 2; jx++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][jx][r] = 0;
    for (int64_t k0 = 0; k0 < k; k0 += 32) {
        const int64_t c = k0 + 16 * h;
        v4i af[2], bf[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            af[t] = load16_masked(ar[t], c, k);
            bf[t] = load16_masked(wr[t], c, k);
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int jx = 0; jx < 2; jx++)
                acc[i][jx] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[jx], acc[i][jx], 0, 0, 0);
    }
#pragma unroll
    for (int jx = 0; jx < 2; jx++) {
        const int64_t col = n0 + 32 * jx + l32;
        if (col >= n) continue;
        const float sw = w_scales[col];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t row = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) {
                    const float sa = act_scales ? act_scales[row] : act_scale;
                    out[row * n + col] = ((float)acc[i][jx][r] * sa) * sw;
                }
            }
    }
}

// ---------------------------------------------------------------------------
// int8 x int8 -> f32, m >= 32 and k a multiple of 64: a 128 x 128 output tile
// per 4-wavefront workgroup (two per CU), each wavefront a 64 x 64 block of
// four v_mfma_i32_32x32x32_i8 tiles.  Both operands (row-major, k
// contiguous) are copied global -> LDS by buffer loads into LDS, 64 k-bytes
// of the tile's 128 activation rows and 128 weight rows per stage, in a ring
// of four stages issued three steps ahead.  A row's four 16-byte chunks sit at
// positions c ^ ((r >> 2) & 3), so the 16-byte reads of 16 consecutive rows
// (64-byte row stride) fall on distinct banks.  Work items are numbered so
// that all m-tiles of one n-tile run on one XCD (workgroups are dealt to the
// 8 XCDs round-robin) and share its L2 copy of the weight rows.
// The i32 sums are exact; out = ((f32)acc * sa) * sw as the crate.
// ---------------------------------------------------------------------------
constexpr int I8T = 128, I8K = 64, I8NST = 4, I8XCD = 8;
constexpr int I8STAGE = 2 * I8T * I8K;  // activation rows, then weight rows
constexpr int I8COPIES = 4;             // copy instructions per wavefront and stage

__global__ __launch_bounds__(256, 2) void int8_gemm_kernel(const int8_t *__restrict__ a, const int8_t *__restrict__ w,
                                                           const float *__restrict__ act_scales, float act_scale,
                                                           const float *__restrict__ w_scales, int m, int n, int k,
                                                           float *__restrict__ out, int ntm, int items, int per_xcd) {
    __shared__ __align__(16) uint8_t lds[I8NST * I8STAGE];
    const int xcd = blockIdx.x % I8XCD, local = blockIdx.x / I8XCD;
    const int item = xcd * per_xcd + local;
    if (local >= per_xcd || item >= items) return;  // uniform over the workgroup
    const int tn = item / ntm, tm = item - tn * ntm;
    const int m0 = tm * I8T, n0 = tn * I8T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, l32 = lane & 31;

    const rsrc_t ra = buf_rsrc(a, (uint32_t)((int64_t)m * k));
    const rsrc_t rw = buf_rsrc(w, (uint32_t)((int64_t)n * k));
    // copy instruction i of this wavefront fills chunks (2*wave + i)*64 + lane
    // of a 128 x 64-byte region: row r = chunk / 4, position chunk % 4
    uint32_t aoff[2], woff[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = (2 * wave + i) * 64 + lane, r = t >> 2, cp = t & 3;
        const int c = cp ^ ((r >> 2) & 3);
        aoff[i] = m0 + r < m ? (uint32_t)((int64_t)(m0 + r) * k + 16 * c) : BUF_OOB;  // rows past m / n read zeros
        woff[i] = n0 + r < n ? (uint32_t)((int64_t)(n0 + r) * k + 16 * c) : BUF_OOB;
    }
    const int nk = k / I8K;
    auto issue = [&](int slot_ks) {
        // stage slot_ks % 4 gets step slot_ks's data; a step past k (issued
        // ahead, never read) reloads the last step, so no copy addresses
        // memory past the rows
        uint8_t *st = lds + (slot_ks & (I8NST - 1)) * I8STAGE;
        const int ks = min(slot_ks, nk - 1);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            buf_to_lds16(ra, st + 1024 * (2 * wave + i), aoff[i], ks * I8K);
            buf_to_lds16(rw, st + I8T * I8K + 1024 * (2 * wave + i), woff[i], ks * I8K);
        }
    };
    auto frag = [&](const uint8_t *base, int R, int s) {  // 16 k-bytes of row R, slice s, half h
        const int C = 2 * s + h;
        return *(const v4i *)(base + R * I8K + 16 * (C ^ ((R >> 2) & 3)));
    };

    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    issue(0);
    issue(1);
    issue(2);
    for (int ks = 0; ks < nk; ks++) {
        wait_vmcnt<2 * I8COPIES>();  // this step's copies have landed (two later steps' may be in flight)
        stage_barrier();             // ... for every wavefront; and step ks - 1's stage is free
        issue(ks + 3);
        const uint8_t *st = lds + (ks & (I8NST - 1)) * I8STAGE;
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            v4i af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                af[t] = frag(st, 64 * wm + 32 * t + l32, s2);
                bf[t] = frag(st + I8T * I8K, 64 * wn + 32 * t + l32, s2);
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();  // no copy may still be landing when the workgroup ends
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = n0 + 64 * wn + 32 * j + l32;
        if (col >= n) continue;
        const float sw = w_scales[col];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < m) {
                    const float sa = act_scales ? act_scales[row] : act_scale;
                    out[(int64_t)row * n + col] = ((float)acc[i][j][r] * sa) * sw;
                }
            }
    }
}

// ---------------------------------------------------------------------------
// quantize_int8_per_token: one workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quantize_int8_per_token_kernel(const float *__restrict__ a, int64_t k,
                                                                      int8_t *__restrict__ q,
                                                                      float *__restrict__ scales) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float *x = a + row * k;
    float mx = 0.0f;
    for (int64_t i = threadIdx.x; i < k; i += 256) mx = fmaxf(mx, fabsf(x[i]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
    if (threadIdx.x == 0) scales[row] = scale;
    for (int64_t i = threadIdx.x; i < k; i += 256) q[row * k + i] = (int8_t)clampi(sat_f2i(roundf(x[i] / scale)), -127, 127);
}

// ---------------------------------------------------------------------------
// Weight-only matmuls, f32 activations (up to 8 rows per pass): one
// wavefront per output column; lane L takes the 32-element groups
// L, L + 64, ...; partials reduced over the wavefront.
//   WQ4: Q4_0-style packed nibbles (16 B per group, low nibble = even k) and
//        one f32 scale per group: group sum of a * (nibble - 8), times scale;
//   WI8: int8 weights, per-column scale applied to the total;
//   WF16: f16 weights.
// ---------------------------------------------------------------------------
enum { WQ4 = 0, WI8 = 1, WF16 = 2 };

template <int WT, int B>
__global__ __launch_bounds__(256) void wonly_kernel(const float *__restrict__ a, const void *__restrict__ wv,
                                                    const float *__restrict__ wscale, int m, int n, int64_t k,
                                                    float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= n) return;  // wave-uniform
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0.0f;
    const int64_t ngf = k / 32;  // full groups
    for (int64_t g = lane; g < ngf; g += 64) {
        float wf[32];
        if (WT == WQ4) {
            const uint8_t *p = (const uint8_t *)wv + j * (k / 2) + g * 16;
            uint32_t pk[4];
            __builtin_memcpy(pk, p, 16);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t byte = (pk[i >> 2] >> (8 * (i & 3))) & 0xffu;
                wf[2 * i] = (float)((int)(byte & 15u) - 8);
                wf[2 * i + 1] = (float)((int)(byte >> 4) - 8);
            }
        } else if (WT == WI8) {
            const int8_t *p = (const int8_t *)wv + j * k + g * 32;
            int8_t t[32];
            __builtin_memcpy(t, p, 32);
#pragma unroll
            for (int i = 0; i < 32; i++) wf[i] = (float)t[i];
        } else {
            const uint16_t *p = (const uint16_t *)wv + j * k + g * 32;
            uint16_t t[32];
            __builtin_memcpy(t, p, 64);
#pragma unroll
            for (int i = 0; i < 32; i++) wf[i] = f16_bits_to_f32(t[i]);
        }
#pragma unroll
        for (int b = 0; b < B; b++) {
            if (b < m) {
                const float *ab = a + (int64_t)b * k + g * 32;
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) s = __builtin_fmaf(ab[i], wf[i], s);
                acc[b] += WT == WQ4 ? s * wscale[j * ngf + g] : s;
            }
        }
    }
    if (WT != WQ4) {  // the K % 32 tail (the int4 formats require K % 32 == 0)
        for (int64_t c = ngf * 32 + lane; c < k; c += 64) {
            const float wf = WT == WI8 ? (float)((const int8_t *)wv)[j * k + c] : f16_bits_to_f32(((const uint16_t *)wv)[j * k + c]);
#pragma unroll
            for (int b = 0; b < B; b++)
                if (b < m) acc[b] = __builtin_fmaf(a[(int64_t)b * k + c], wf, acc[b]);
        }
    }
#pragma unroll
    for (int b = 0; b < B; b++) {
        if (b < m) {
            const float s = wave_sum(acc[b]);
            if (lane == 0) out[(int64_t)b * n + j] = WT == WI8 ? s * wscale[j] : s;
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_0 x Q8 GEMV (int4_matmul_gemv_q4_x_q8_neon): the activation is
// quantised per group of 32 (f32 scale, i8) into even / odd halves (the
// order of the packed nibbles) plus the group's quant sum; then per column
// and group the exact dot  sum (nibble - 8) * q = dot4(nibbles, q) - 8 * sum(q),
// total += ((f32)dot * w_scale) * a_scale.
// Activation record per group: 16 even quants, 16 odd quants, i32 sum, f32 scale.
// ---------------------------------------------------------------------------
constexpr int Q8G_BYTES = 40;

__global__ __launch_bounds__(256) void quantize_q8_groups_kernel(const float *__restrict__ a, int64_t k,
                                                                 uint8_t *__restrict__ rec, int8_t *__restrict__ q_out,
                                                                 float *__restrict__ s_out) {
    // eight lanes per group, four elements each
    const int64_t gi = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    const int64_t ng = k / 32;
    const bool ok = gi < ng;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (ok) __builtin_memcpy(v, a + gi * 32 + 4 * sub, 16);
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    mx = fmaxf(mx, __shfl_xor(mx, 4));
    const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    int q[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float r = roundf(v[i] * inv);
        q[i] = r != r ? 0 : (int)fminf(fmaxf(r, -128.0f), 127.0f);
        sum += q[i];
    }
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (!ok) return;
    uint8_t *r = rec + gi * Q8G_BYTES;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = 4 * sub + i;  // element of the group
        r[(e & 1) * 16 + (e >> 1)] = (uint8_t)(int8_t)q[i];
        if (q_out) q_out[gi * 32 + e] = (int8_t)q[i];
    }
    if (sub == 0) {
        *(int32_t *)(r + 32) = sum;
        *(float *)(r + 36) = scale;
        if (s_out) s_out[gi] = scale;
    }
}

__global__ __launch_bounds__(256) void q4_x_q8_gemv_kernel(const uint8_t *__restrict__ wp, const float *__restrict__ ws,
                                                           const uint8_t *__restrict__ rec, int n, int64_t k,
                                                           float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= n) return;  // wave-uniform
    const int64_t ng = k / 32;
    float total = 0.0f;
    for (int64_t g = lane; g < ng; g += 64) {
        uint32_t pk[4];
        __builtin_memcpy(pk, wp + j * (k / 2) + g * 16, 16);
        const uint8_t *r = rec + g * Q8G_BYTES;
        int ev[4], od[4];
        __builtin_memcpy(ev, r, 16);
        __builtin_memcpy(od, r + 16, 16);
        int dot = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            dot = sdot4((int)(pk[i] & 0x0F0F0F0Fu), ev[i], dot);
            dot = sdot4((int)((pk[i] >> 4) & 0x0F0F0F0Fu), od[i], dot);
        }
        dot -= 8 * *(const int32_t *)(r + 32);
        total += ((float)dot * ws[j * ng + g]) * *(const float *)(r + 36);
    }
    total = wave_sum(total);
    if (lane == 0) out[j] = total;
}

// ---------------------------------------------------------------------------
// quantize_int4_q4_0: one thread per group of 32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quantize_int4_q4_0_kernel(const float *__restrict__ w, int64_t n, int64_t k,
                                                                 uint8_t *__restrict__ packed,
                                                                 float *__restrict__ scales) {
    const int64_t ng = k / 32;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n * ng) return;
    const int64_t row = t / ng, g = t - row * ng;
    const float *x = w + row * k + g * 32;
    float mx = 0.0f;
    for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(x[i]));
    const float scale = mx > 0.0f ? mx / 7.0f : 1.0f;
    scales[t] = scale;
    uint8_t *o = packed + row * (k / 2) + g * 16;
    for (int j = 0; j < 16; j++) {
        const int ql = clampi(sat_f2i(roundf(x[2 * j] / scale)), -8, 7) + 8;
        const int qh = clampi(sat_f2i(roundf(x[2 * j + 1] / scale)), -8, 7) + 8;
        o[j] = (uint8_t)((qh << 4) | ql);
    }
}

// ---------------------------------------------------------------------------
// Dequantizers: one thread per output element.
// ---------------------------------------------------------------------------
// The crate's Q6_K dequantizer (shape_ops.rs:2848-2899), including its
// sub-scale index 8h + {0,2,4,6} for all 32 elements of a group.
__global__ __launch_bounds__(256) void dequant_q6k_crate_kernel(const uint8_t *__restrict__ in, int64_t nel,
                                                                float *__restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nel) return;
    const int64_t b = e >> 8;
    const int i = (int)(e & 255), hh = i >> 7, gq = (i >> 5) & 3, l = i & 31;
    const uint8_t *blk = in + b * 210;
    const uint8_t *ql = blk + hh * 64, *qh = blk + 128 + hh * 32;
    const int8_t *sc = (const int8_t *)(blk + 192) + hh * 8;
    const int qhi = qh[l];
    const int lowbits = gq == 0 ? (ql[l] & 0xF) : gq == 1 ? (ql[l + 32] & 0xF) : gq == 2 ? (ql[l] >> 4) : (ql[l + 32] >> 4);
    const int q = (lowbits | (((qhi >> (2 * gq)) & 3) << 4)) - 32;
    const float d = f16_bits_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
    out[e] = d * (float)(sc[2 * gq] * q);
}

// rows[r] of a Q4_0-style table ([N][K/2] packed, [N][K/32] scales) -> out[r][K]
// (a row index outside 0..ntab-1 yields zeros)
__global__ __launch_bounds__(256) void q4_0_rows_kernel(const uint8_t *__restrict__ packed, const float *__restrict__ scales,
                                                        int64_t ntab, const int64_t *__restrict__ rows, int64_t nr,
                                                        int64_t k, float *__restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nr * k) return;
    const int64_t r = e / k, c = e - r * k;
    const int64_t row = rows[r];
    if (row < 0 || row >= ntab) {
        out[e] = 0.0f;
        return;
    }
    const uint8_t byte = packed[row * (k / 2) + (c >> 1)];
    const int v = (c & 1) ? (byte >> 4) - 8 : (byte & 15) - 8;
    out[e] = (float)v * scales[row * (k / 32) + (c >> 5)];
}

// rows[r] of an int8 table ([N][K] i8, [N][K/32] scales) -> out[r][K]
__global__ __launch_bounds__(256) void q8_0_rows_kernel(const int8_t *__restrict__ w, const float *__restrict__ scales,
                                                        int64_t ntab, const int64_t *__restrict__ rows, int64_t nr,
                                                        int64_t k, float *__restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nr * k) return;
    const int64_t r = e / k, c = e - r * k;
    const int64_t row = rows[r];
    if (row < 0 || row >= ntab) {
        out[e] = 0.0f;
        return;
    }
    out[e] = (float)w[row * k + c] * scales[row * (k / 32) + (c >> 5)];
}

unsigned blocks_for(int64_t items, int per) { return (unsigned)((items + per - 1) / per); }

template <int B>
hipError_t launch_int8_rows(const int8_t *a, const int8_t *w, const float *as, float asc, const float *ws, int m, int n,
                            int64_t k, float *out, hipStream_t s) {
    int8_rows_kernel<B><<<blocks_for(n, 4), 256, 0, s>>>(a, w, as, asc, ws, m, n, k, out);
    return hipGetLastError();
}

template <int WT, int B>
hipError_t launch_wonly_b(const float *a, const void *w, const float *ws, int m, int n, int64_t k, float *out,
                          hipStream_t s) {
    wonly_kernel<WT, B><<<blocks_for(n, 4), 256, 0, s>>>(a, w, ws, m, n, k, out);
    return hipGetLastError();
}

template <int WT>
hipError_t launch_wonly_pass(int B, const float *a, const void *w, const float *ws, int m, int n, int64_t k, float *out,
                             hipStream_t s) {
    switch (B) {
    case 1: return launch_wonly_b<WT, 1>(a, w, ws, m, n, k, out, s);
    case 2: return launch_wonly_b<WT, 2>(a, w, ws, m, n, k, out, s);
    case 4: return launch_wonly_b<WT, 4>(a, w, ws, m, n, k, out, s);
    default: return launch_wonly_b<WT, 8>(a, w, ws, m, n, k, out, s);
    }
}

bool dims_ok(int64_t m, int64_t n, int64_t k) { return m >= 0 && n > 0 && k > 0 && m <= 0x7fffffff && n <= 0x7fffffff; }

}  // namespace

hipError_t launch_int8_matmul(const int8_t *a, const int8_t *w, const float *act_scales, float act_scale,
                              const float *w_scales, int64_t m, int64_t n, int64_t k, float *out, hipStream_t s) {
    if (!a || !w || !w_scales || !out || !dims_ok(m, n, k)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    if (m >= 32 && k % I8K == 0 && k <= 0x7fffffff && m * k < ((int64_t)1 << 31) && n * k < ((int64_t)1 << 31)) {
        const int ntm = (int)blocks_for(m, I8T), ntn = (int)blocks_for(n, I8T);
        const int items = ntm * ntn, per_xcd = (items + I8XCD - 1) / I8XCD;
        int8_gemm_kernel<<<(unsigned)(per_xcd * I8XCD), 256, 0, s>>>(a, w, act_scales, act_scale, w_scales, (int)m,
                                                                     (int)n, (int)k, out, ntm, items, per_xcd);
        return hipGetLastError();
    }
    if (m >= 32) {
        const dim3 grid(blocks_for(n, 128), blocks_for(m, 128));
        if (grid.y > 65535) return hipErrorInvalidValue;
        int8_mfma_kernel<<<grid, 256, 0, s>>>(a, w, act_scales, act_scale, w_scales, (int)m, (int)n, k, out);
        return hipGetLastError();
    }
    for (int64_t r0 = 0; r0 < m; r0 += 8) {
        const int mb = (int)(m - r0 < 8 ? m - r0 : 8);
        const int8_t *ar = a + r0 * k;
        const float *asr = act_scales ? act_scales + r0 : nullptr;
        float *o = out + r0 * n;
        hipError_t e = mb == 1   ? launch_int8_rows<1>(ar, w, asr, act_scale, w_scales, mb, (int)n, k, o, s)
                       : mb <= 2 ? launch_int8_rows<2>(ar, w, asr, act_scale, w_scales, mb, (int)n, k, o, s)
                       : mb <= 4 ? launch_int8_rows<4>(ar, w, asr, act_scale, w_scales, mb, (int)n, k, o, s)
                                 : launch_int8_rows<8>(ar, w, asr, act_scale, w_scales, mb, (int)n, k, o, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_quantize_int8_per_token(const float *a, int64_t m, int64_t k, int8_t *q, float *scales,
                                          hipStream_t s) {
    if (!a || !q || !scales || m < 0 || k <= 0 || m > 0x7fffffff) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    quantize_int8_per_token_kernel<<<(unsigned)m, 256, 0, s>>>(a, k, q, scales);
    return hipGetLastError();
}

hipError_t launch_weight_only_matmul(int wt, const float *a, const void *w, const float *w_scales, int64_t m, int64_t n,
                                     int64_t k, float *out, hipStream_t s) {
    if (!a || !w || !out || !dims_ok(m, n, k)) return hipErrorInvalidValue;
    if (wt == CRATE_W_Q4_0 && (k % 32 || !w_scales)) return hipErrorInvalidValue;
    if (wt == CRATE_W_I8 && !w_scales) return hipErrorInvalidValue;
    if (wt != CRATE_W_Q4_0 && wt != CRATE_W_I8 && wt != CRATE_W_F16) return hipErrorInvalidValue;
    for (int64_t r0 = 0; r0 < m; r0 += 8) {
        const int mb = (int)(m - r0 < 8 ? m - r0 : 8);
        const int B = mb == 1 ? 1 : mb <= 2 ? 2 : mb <= 4 ? 4 : 8;
        hipError_t e;
        if (wt == CRATE_W_Q4_0) e = launch_wonly_pass<WQ4>(B, a + r0 * k, w, w_scales, mb, (int)n, k, out + r0 * n, s);
        else if (wt == CRATE_W_I8) e = launch_wonly_pass<WI8>(B, a + r0 * k, w, w_scales, mb, (int)n, k, out + r0 * n, s);
        else e = launch_wonly_pass<WF16>(B, a + r0 * k, w, nullptr, mb, (int)n, k, out + r0 * n, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

size_t q4_x_q8_act_bytes(int64_t k) { return align_up((size_t)(k / 32) * Q8G_BYTES, 256); }

hipError_t launch_q4_x_q8_gemv(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n, int64_t k,
                               float *out, void *act, int8_t *q_out, float *s_out, hipStream_t s) {
    if (!a || !w_packed || !w_scales || !out || !act || n <= 0 || k <= 0 || k % 32 || n > 0x7fffffff)
        return hipErrorInvalidValue;
    const int64_t ng = k / 32;
    quantize_q8_groups_kernel<<<blocks_for(ng, 32), 256, 0, s>>>(a, k, (uint8_t *)act, q_out, s_out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    q4_x_q8_gemv_kernel<<<blocks_for(n, 4), 256, 0, s>>>(w_packed, w_scales, (const uint8_t *)act, (int)n, k, out);
    return hipGetLastError();
}

hipError_t launch_quantize_int4_q4_0(const float *w, int64_t n, int64_t k, uint8_t *packed, float *scales,
                                     hipStream_t s) {
    if (!w || !packed || !scales || n <= 0 || k <= 0 || k % 32) return hipErrorInvalidValue;
    quantize_int4_q4_0_kernel<<<blocks_for(n * (k / 32), 256), 256, 0, s>>>(w, n, k, packed, scales);
    return hipGetLastError();
}

hipError_t launch_dequantize_q6_k_crate(const uint8_t *blocks, int64_t nel, float *out, hipStream_t s) {
    if (!blocks || !out || nel <= 0 || nel % 256) return hipErrorInvalidValue;
    dequant_q6k_crate_kernel<<<blocks_for(nel, 256), 256, 0, s>>>(blocks, nel, out);
    return hipGetLastError();
}

hipError_t launch_dequant_rows(int wt, const void *table, const float *scales, int64_t ntab, const int64_t *rows,
                               int64_t nr, int64_t k, float *out, hipStream_t s) {
    if (!table || !scales || !rows || !out || nr < 0 || ntab <= 0 || k <= 0 || k % 32) return hipErrorInvalidValue;
    if (nr == 0) return hipSuccess;
    if (wt == CRATE_W_Q4_0)
        q4_0_rows_kernel<<<blocks_for(nr * k, 256), 256, 0, s>>>((const uint8_t *)table, scales, ntab, rows, nr, k, out);
    else if (wt == CRATE_W_I8)
        q8_0_rows_kernel<<<blocks_for(nr * k, 256), 256, 0, s>>>((const int8_t *)table, scales, ntab, rows, nr, k, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace aq
