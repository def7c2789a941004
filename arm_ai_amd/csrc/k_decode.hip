// k_decode.hip -- the f32 operations between the quantized matmuls of one
// Llama decode step (one token at a device-resident position), as fused
// gfx950 kernels, so a captured decode step is ~9 launches per layer instead
// of ~30 framework ops.  They follow candle-transformers 0.8.4
// quantized_llama, which native/arm_ai_nif/src/llama_candle.rs:119 runs per
// generated token:
//   embedding lookup; per layer h = x + wo(attn(rms_norm(x))),
//   x = h + w2(silu(w1(n)) * w3(n)) with n = rms_norm(h); final rms_norm;
//   rms_norm(x) = x / sqrt(mean(x^2) + eps) * w; silu(x) = x / (1 + e^-x);
//   attention: rope_i (interleaved pairs) on q and k at the position, k and v
//   appended to the cache, each query head attending to its group's kv head
//   (n_head / n_kv_head queries per kv head), softmax(q.k / sqrt(d)) . v,
//   no mask for a single query position;
//   next token = first index of the largest logit (llama_candle.rs:154-176).
// All arithmetic is IEEE f32 (the library is built without fast-math); sums
// are reordered relative to candle's CPU loops, so results agree within
// rounding, not bit for bit.
#include "aq_internal.h"

namespace aq {

namespace {

constexpr int DEC_THREADS = 256;   // row kernels (embedding, RMSNorm, SiLU)
constexpr int WIDE_THREADS = 1024; // one-workgroup kernels that stream a long vector (attention, argmax)

// Sum / max over a block of NT threads (NT/64 wavefronts); every thread gets
// the result.  red: NT/64 floats of LDS.  The leading barrier lets red be
// reused by consecutive calls; the trailing one publishes it (and any LDS
// written before the call).
template <int NT>
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) s += red[w];
    return s;
}
template <int NT>
__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) s = fmaxf(s, red[w]);
    return s;
}

// out row r = embedding row d_tok[r] (a token id outside [0, vocab) gives
// zeros); one workgroup per row.  hidden % 4 == 0 (checked by the launcher):
// float4 copies.
__global__ __launch_bounds__(DEC_THREADS) void embed_kernel(const float *__restrict__ table, int64_t vocab,
                                                            const int64_t *__restrict__ d_tok, int hidden,
                                                            float *__restrict__ out) {
    const int64_t t = d_tok[blockIdx.x];
    const bool ok = t >= 0 && t < vocab;
    const float4 *src = (const float4 *)(table + (ok ? t : 0) * hidden);
    float4 *dst = (float4 *)(out + (int64_t)blockIdx.x * hidden);
    for (int i = threadIdx.x; i < hidden / 4; i += DEC_THREADS)
        dst[i] = ok ? src[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// One row per workgroup: x += delta (when delta is given, written back to x:
// the residual stream), then out = x / sqrt(sum(x^2)/n + eps) * w.  The row
// (n % 4 == 0, n <= 4 * RMS_V * DEC_THREADS) is held in registers, so x is
// read once and every load is issued before the first use.  The body is
// shared by the kernel that quantises the result in the same launch
// (rmsnorm_act_kernel), so both produce the same values bit for bit: `put`
// receives float4 i = threadIdx.x + j * DEC_THREADS of the output row.
constexpr int RMS_V = 8;
template <typename Put>
__device__ __forceinline__ void rmsnorm_row(float *__restrict__ x, const float *__restrict__ delta,
                                            const float *__restrict__ w, int n, float eps, float *red, Put put) {
    float4 *xr = (float4 *)(x + (int64_t)blockIdx.x * n);
    const float4 *dr = delta ? (const float4 *)(delta + (int64_t)blockIdx.x * n) : nullptr;
    const float4 *w4 = (const float4 *)w;
    const int n4 = n / 4;
    float4 v[RMS_V], d[RMS_V];
#pragma unroll
    for (int j = 0; j < RMS_V; j++) {
        const int i = threadIdx.x + j * DEC_THREADS;
        v[j] = i < n4 ? xr[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        d[j] = (dr && i < n4) ? dr[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < RMS_V; j++) {
        const int i = threadIdx.x + j * DEC_THREADS;
        if (dr) {
            v[j].x += d[j].x;
            v[j].y += d[j].y;
            v[j].z += d[j].z;
            v[j].w += d[j].w;
            if (i < n4) xr[i] = v[j];
        }
        ss = __builtin_fmaf(v[j].x, v[j].x, ss);
        ss = __builtin_fmaf(v[j].y, v[j].y, ss);
        ss = __builtin_fmaf(v[j].z, v[j].z, ss);
        ss = __builtin_fmaf(v[j].w, v[j].w, ss);
    }
    const float m = sqrtf(block_sum<DEC_THREADS>(ss, red) / (float)n + eps);
#pragma unroll
    for (int j = 0; j < RMS_V; j++) {
        const int i = threadIdx.x + j * DEC_THREADS;
        if (i < n4) {
            const float4 ww = w4[i];
            put(j, i, make_float4((v[j].x / m) * ww.x, (v[j].y / m) * ww.y, (v[j].z / m) * ww.z, (v[j].w / m) * ww.w));
        }
    }
}

__global__ __launch_bounds__(DEC_THREADS) void rmsnorm_kernel(float *__restrict__ x, const float *__restrict__ delta,
                                                              const float *__restrict__ w, int n, float eps,
                                                              float *__restrict__ out) {
    __shared__ float red[DEC_THREADS / 64];
    float4 *orow = (float4 *)(out + (int64_t)blockIdx.x * n);
    rmsnorm_row(x, delta, w, n, eps, red, [&](int, int i, float4 h) { orow[i] = h; });
}

// rmsnorm_kernel's output quantised to Q8_K in the same launch (the prompt's
// norm before a prefill GEMM).  Float4 i = threadIdx.x + j * DEC_THREADS of
// the row is held by lane l of wavefront w (threadIdx.x = 64 w + l), so
// wavefront w holds Q8_K block w + 4j whole, four values a lane: each
// wavefront quantises its blocks from registers with the quantizer's
// one-wavefront code (q8k_block_wave, the arithmetic of the quantizer
// kernel's), with no LDS and no barrier after the norm.  out, when given,
// gets the normed row.
__global__ __launch_bounds__(DEC_THREADS) void rmsnorm_act_kernel(float *__restrict__ x,
                                                                  const float *__restrict__ delta,
                                                                  const float *__restrict__ w, int n, float eps,
                                                                  float *__restrict__ out, ActPlanes a) {
    static_assert(DEC_THREADS == 256, "wavefront w holds blocks w + 4j");
    __shared__ float red[DEC_THREADS / 64];
    float4 *orow = out ? (float4 *)(out + (int64_t)blockIdx.x * n) : nullptr;
    float4 hv[RMS_V];
    rmsnorm_row(x, delta, w, n, eps, red, [&](int j, int i, float4 h) {
        hv[j] = h;
        if (orow) orow[i] = h;
    });
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nb = n / QK_K;
#pragma unroll
    for (int j = 0; j < RMS_V; j++) {
        const int b = wave + 4 * j;
        if (b >= nb) break;  // uniform over the wavefront
        const float v[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
        int bsum;
        float d;
        const uint32_t packed = q8k_block_wave(v, lane, &bsum, &d);
        store_q8k_block64(a, blockIdx.x, n, b, lane, packed, bsum, d);
    }
}

// out[r][i] = silu(g[r][i]) * u[r][i] for rows r (grid y) of n; row r of g
// and u starts at r * ld (the merged w1|w3 output: u = g + n, ld = 2n).
__global__ __launch_bounds__(DEC_THREADS) void silu_mul_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                               int64_t ld, int64_t n, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * DEC_THREADS + threadIdx.x;
    if (i >= n) return;
    const int64_t r = blockIdx.y;
    const float gv = g[r * ld + i];
    out[r * n + i] = (gv / (1.0f + expf(-gv))) * u[r * ld + i];
}

// out[r][i] = silu(g) * u for the output row r (grid y) of a weight whose
// rows are gate and up rows in pairs of four (row 8b + j: gate row 4b + j
// for j < 4, up row 4b + j - 4 after): g = y[r][8(i/4) + i%4], u four places
// on.  n (a multiple of 4) outputs per row; row r of y starts at r * ld.
__global__ __launch_bounds__(DEC_THREADS) void swiglu_pairs_kernel(const float *__restrict__ y, int64_t ld, int64_t n,
                                                                   float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * DEC_THREADS + threadIdx.x;
    if (i >= n) return;
    const int64_t r = blockIdx.y;
    const int64_t j = r * ld + 8 * (i >> 2) + (i & 3);
    const float gv = y[j];
    out[r * n + i] = (gv / (1.0f + expf(-gv))) * y[j + 4];
}

// swiglu_pairs_kernel's values quantised to Q8_K in the same launch: grid
// (ceil(n / 1024), m) workgroups, a wavefront per block of 256 values (no
// workgroup takes more blocks than another, no LDS, no barrier).  Lane l
// forms values 4l .. 4l + 3 of its block by swiglu_pairs_kernel's
// expression from the 32 bytes 8l .. 8l + 7 of the block's 512 paired
// columns (the gate four, then the up four), and the wavefront quantises
// the block with the quantizer's 64-lane code (q8k_block_wave, the same
// bytes as the per-block kernel).  y 16-byte aligned, ld a multiple of 4
// (checked by the launcher).
__global__ __launch_bounds__(DEC_THREADS) void swiglu_pairs_act_kernel(const float *__restrict__ y, int64_t ld, int n,
                                                                       float *__restrict__ out, ActPlanes a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.x * (DEC_THREADS / 64) + wave;  // this wavefront's block
    const int64_t r = blockIdx.y;
    if (b >= n / QK_K) return;  // uniform over the wavefront
    const float4 *src = (const float4 *)(y + r * ld + 2 * (int64_t)b * QK_K + 8 * lane);
    const float4 g = src[0], u = src[1];
    float v[4];
    v[0] = (g.x / (1.0f + expf(-g.x))) * u.x;
    v[1] = (g.y / (1.0f + expf(-g.y))) * u.y;
    v[2] = (g.z / (1.0f + expf(-g.z))) * u.z;
    v[3] = (g.w / (1.0f + expf(-g.w))) * u.w;
    if (out) *(float4 *)(out + r * n + (int64_t)b * QK_K + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
    int bsum;
    float d;
    const uint32_t packed = q8k_block_wave(v, lane, &bsum, &d);
    store_q8k_block64(a, r, n, b, lane, packed, bsum, d);
}

// Sum over aligned groups of N lanes (N = 2, 4, 8, 16, 32 or 64), every lane
// of a group getting the same value: DPP moves within 16-lane rows (quad
// swaps, half-row mirror, row rotations), cross-lane permutes only between
// rows.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return u32_as_f32((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f32_as_u32(v), CTRL, 0xF, 0xF, false));
}
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group of 2..64 lanes");
    if (N >= 16) {
        v += dpp_f<0x128>(v);  // row_ror:8
        v += dpp_f<0x124>(v);  // row_ror:4
    } else if (N == 8) {
        v += dpp_f<0x141>(v);  // row_half_mirror: lanes l and 7 - l of each half row
    }
    if (N >= 4) v += dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
    v += dpp_f<0xB1>(v);              // quad_perm [1,0,3,2]
    if (N >= 32) v += __shfl_xor(v, 16);
    if (N >= 64) v += __shfl_xor(v, 32);
    return v;
}

// Attention for one query position at *d_pos, one 1024-thread workgroup per
// query head.  qk = [q (n_head*hd) | k (n_kv*hd)] before rotation, v
// (n_kv*hd); the caches are [n_kv][max_seq][hd] for this layer.  Each
// workgroup rotates its q head and its group's k (rope_i: pairs (2i, 2i+1) by
// pos * theta_i, from the cos/sin tables [max_seq][hd/2]); the first
// workgroup of each group stores the rotated k and v at pos for later steps,
// and every workgroup uses its own LDS copy for position pos, so no
// workgroup waits for another.
//   scores: HD4 = hd/4 lanes per position, each a float4 of q and of k_p, the
//     partial dots summed over the lanes (coalesced 1 KB key reads);
//   softmax: block max, e_p = exp(s_p - max), block sum;
//   output: thread (d4, g) sums positions p = g (mod 4096/hd) of e_p * v_p[d]
//     for four consecutive d (float4 reads), the groups' partials are summed
//     in LDS in two levels, and the result is divided by the sum of the e_p.
// The value rows do not depend on the scores: each thread's first ones are
// loaded before the softmax's barriers.
constexpr int ATT_MAX_SEQ = 8192;
constexpr int ATT_MAX_HD = 256;
template <int HD4>
__global__ __launch_bounds__(WIDE_THREADS) void attn_decode_kernel(
    const float *__restrict__ qk, const float *__restrict__ v, const float *__restrict__ cosb,
    const float *__restrict__ sinb, const int64_t *__restrict__ d_pos, float *__restrict__ kc, float *__restrict__ vc,
    int n_head, int n_kv, int max_seq, float *__restrict__ out) {
    constexpr int hd = 4 * HD4;
    // value rows loaded ahead into registers, in flight across the softmax
    // (fewer for wide heads: a 1024-thread workgroup has 128 VGPRs per lane)
    constexpr int VPRE = HD4 <= 16 ? 8 : 4;
    constexpr int G = WIDE_THREADS / HD4;    // position groups of the output pass
    __shared__ __align__(16) float qs[hd];
    __shared__ __align__(16) float ks[hd];
    __shared__ __align__(16) float vs[hd];
    __shared__ float sc[ATT_MAX_SEQ];
    __shared__ float red[WIDE_THREADS / 64];
    __shared__ float4 part4[WIDE_THREADS];
    __shared__ float4 sc4[16 * HD4];
    const int head = blockIdx.x, tid = threadIdx.x;
    const int rep = n_head / n_kv, kvh = head / rep;
    const int pos = (int)*d_pos;
    if (pos < 0 || pos >= max_seq) return;  // uniform; the host checks, this never indexes out of the cache
    const float *q0 = qk + (int64_t)head * hd;
    const float *k0 = qk + (int64_t)n_head * hd + (int64_t)kvh * hd;
    const float *v0 = v + (int64_t)kvh * hd;
    const float *cr = cosb + (int64_t)pos * (hd / 2), *sr = sinb + (int64_t)pos * (hd / 2);
    float *kh = kc + (int64_t)kvh * max_seq * hd;
    float *vh = vc + (int64_t)kvh * max_seq * hd;

    // rotation inputs
    float ra = 0.0f, rb = 0.0f, rka = 0.0f, rkb = 0.0f, rc = 0.0f, rsn = 0.0f, rv = 0.0f;
    if (tid < hd / 2) {
        rc = cr[tid];
        rsn = sr[tid];
        ra = q0[2 * tid];
        rb = q0[2 * tid + 1];
        rka = k0[2 * tid];
        rkb = k0[2 * tid + 1];
    } else if (tid >= 512 && tid < 512 + hd) {
        rv = v0[tid - 512];
    }
    if (tid < hd / 2) {
        qs[2 * tid] = ra * rc - rb * rsn;
        qs[2 * tid + 1] = ra * rsn + rb * rc;
        ks[2 * tid] = rka * rc - rkb * rsn;
        ks[2 * tid + 1] = rka * rsn + rkb * rc;
    } else if (tid >= 512 && tid < 512 + hd) {
        vs[tid - 512] = rv;
    }
    __syncthreads();
    if (head % rep == 0 && tid < hd) {
        kh[(int64_t)pos * hd + tid] = ks[tid];
        vh[(int64_t)pos * hd + tid] = vs[tid];
    }

    // scores q . k_p / sqrt(hd), p = 0..pos: HD4 lanes share a key row (lane
    // c holds float4 c of q), so one load instruction reads 64 / HD4
    // consecutive rows, 1 KB contiguous; the row's dot is summed over its
    // lanes by a butterfly within the lane group
    constexpr int RPI = 64 / HD4;  // rows per load instruction
    constexpr int SU_K = 4;        // rows per lane with loads in flight together
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane % HD4;
    const float4 qv = ((const float4 *)qs)[c];
    const float4 *kpos = (const float4 *)ks;
    const float rs = sqrtf((float)hd);
    float mx = -INFINITY;
    for (int p0 = wave * RPI + lane / HD4; p0 <= pos; p0 += SU_K * (WIDE_THREADS / 64) * RPI) {
        float4 kv[SU_K];
#pragma unroll
        for (int u = 0; u < SU_K; u++) {
            const int p = p0 + u * (WIDE_THREADS / 64) * RPI;
            kv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p < pos) kv[u] = ((const float4 *)(kh + (int64_t)p * hd))[c];
            else if (p == pos) kv[u] = kpos[c];
        }
#pragma unroll
        for (int u = 0; u < SU_K; u++) {
            const int p = p0 + u * (WIDE_THREADS / 64) * RPI;
            float d = __builtin_fmaf(qv.x, kv[u].x, __builtin_fmaf(qv.y, kv[u].y,
                      __builtin_fmaf(qv.z, kv[u].z, qv.w * kv[u].w)));
            d = lane_group_sum<HD4>(d);
            if (p <= pos) {
                const float sv = d / rs;
                if (c == 0) sc[p] = sv;
                mx = fmaxf(mx, sv);
            }
        }
    }

    // the output pass's first value rows, in flight across the softmax
    const int d4 = tid % HD4, g = tid / HD4;
    float4 vp4[VPRE];
#pragma unroll
    for (int u = 0; u < VPRE; u++) {
        const int p = g + u * G;
        vp4[u] = p < pos ? *(const float4 *)(vh + (int64_t)p * hd + 4 * d4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    mx = block_max<WIDE_THREADS>(mx, red);  // its barriers publish sc[]
    float sum = 0.0f;
    for (int p = tid; p <= pos; p += WIDE_THREADS) {
        const float e = expf(sc[p] - mx);
        sc[p] = e;
        sum += e;
    }
    sum = block_sum<WIDE_THREADS>(sum, red);  // ... and the e_p

    // output: thread (d4, g) takes dims 4*d4..4*d4+3 of positions p = g (mod G)
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto axpy = [&](float w, const float4 x) {
        acc.x = __builtin_fmaf(w, x.x, acc.x);
        acc.y = __builtin_fmaf(w, x.y, acc.y);
        acc.z = __builtin_fmaf(w, x.z, acc.z);
        acc.w = __builtin_fmaf(w, x.w, acc.w);
    };
#pragma unroll
    for (int u = 0; u < VPRE; u++) {
        const int p = g + u * G;
        if (p < pos) axpy(sc[p], vp4[u]);
        else if (p == pos) axpy(sc[p], *(const float4 *)(vs + 4 * d4));
    }
    constexpr int SU = 4;  // positions per thread with loads in flight together
    for (int p0 = g + VPRE * G; p0 <= pos; p0 += SU * G) {
        float4 v4[SU];
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int p = p0 + u * G;
            v4[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p < pos) v4[u] = *(const float4 *)(vh + (int64_t)p * hd + 4 * d4);
            else if (p == pos) v4[u] = *(const float4 *)(vs + 4 * d4);
        }
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int p = p0 + u * G;
            axpy(p <= pos ? sc[p] : 0.0f, v4[u]);
        }
    }
    part4[tid] = acc;
    __syncthreads();
    // sum the G groups: 16 threads per float4 column first add G/16 groups each
    // (G is a multiple of 16: hd <= 256), then 64-thread columns add the 16 results
    if (tid < 16 * HD4) {
        const int c4 = tid % HD4, sl = tid / HD4, per = G / 16;
        float4 t = part4[(sl * per) * HD4 + c4];
        for (int j = 1; j < per; j++) {
            const float4 u4 = part4[(sl * per + j) * HD4 + c4];
            t.x += u4.x;
            t.y += u4.y;
            t.z += u4.z;
            t.w += u4.w;
        }
        sc4[tid] = t;
    }
    __syncthreads();
    if (tid < hd) {
        const int dd = tid >> 2, c = tid & 3;
        float o = 0.0f;
        for (int sl = 0; sl < 16; sl++) {
            const float4 t4 = sc4[sl * HD4 + dd];
            o += c == 0 ? t4.x : c == 1 ? t4.y : c == 2 ? t4.z : t4.w;
        }
        out[(int64_t)head * hd + tid] = o / sum;
    }
}

// Greedy pick: the first index of the largest value (a NaN never wins; all
// NaN gives 0).  Writes it to *d_tok (the next step's input), to
// hist[*d_pos] when hist is given, and advances *d_pos by one.  One
// 1024-thread workgroup, float4 loads (x 16-byte aligned), eight per thread
// in flight (one round trip up to 32768 values); the last n % 4 elements are
// read one by one, and the position is loaded with the first round.
__device__ __forceinline__ void better(float v, int i, float &best, int &idx) {
    if (v > best || (v == best && i < idx)) {  // NaN compares false
        best = v;
        idx = i;
    }
}
__global__ __launch_bounds__(WIDE_THREADS) void argmax_kernel(const float *__restrict__ x, int n,
                                                              int64_t *__restrict__ d_tok, int64_t *__restrict__ d_pos,
                                                              int64_t *__restrict__ hist, int64_t hist_len) {
    __shared__ float bv[WIDE_THREADS / 64];
    __shared__ int bi[WIDE_THREADS / 64];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    const float4 *x4 = (const float4 *)x;
    const int n4 = n / 4;
    const int64_t pos = threadIdx.x == 0 ? *d_pos : 0;  // only thread 0 uses it
    for (int i0 = threadIdx.x; i0 < n4; i0 += 8 * WIDE_THREADS) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * WIDE_THREADS;
            v[u] = i < n4 ? x4[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = 4 * (i0 + u * WIDE_THREADS);
            better(v[u].x, i, best, idx);
            better(v[u].y, i + 1, best, idx);
            better(v[u].z, i + 2, best, idx);
            better(v[u].w, i + 3, best, idx);
        }
    }
    if ((int)threadIdx.x < (n & 3)) better(x[4 * n4 + threadIdx.x], 4 * n4 + (int)threadIdx.x, best, idx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        better(ov, oi, best, idx);
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < WIDE_THREADS / 64; w++) better(bv[w], bi[w], best, idx);
        if (idx == 0x7fffffff) idx = 0;
        *d_tok = idx;
        if (hist && pos >= 0 && pos < hist_len) hist[pos] = idx;
        *d_pos = pos + 1;
    }
}

// The greedy pick from per-workgroup (value bits, row) pairs that a
// matvec's workgroups left (each the first row of its largest value), with
// argmax_kernel's rule: the first row of the largest value, a NaN never
// wins, none at all gives 0; then token, history and position as there, and
// the token's embedding row (table [vocab][hidden], hidden % 4 == 0) to xout
// -- the next step's input.  One 256-thread workgroup.
__global__ __launch_bounds__(DEC_THREADS) void argmax_parts_embed_kernel(
    const int2 *__restrict__ parts, int nparts, int64_t *__restrict__ d_tok, int64_t *__restrict__ d_pos,
    int64_t *__restrict__ hist, int64_t hist_len, const float *__restrict__ table, int64_t vocab, int hidden,
    float *__restrict__ xout) {
    __shared__ float bv[DEC_THREADS / 64];
    __shared__ int bi[DEC_THREADS / 64];
    __shared__ int tok;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    const int64_t pos = threadIdx.x == 0 ? *d_pos : 0;  // only thread 0 uses it
    for (int i = threadIdx.x; i < nparts; i += DEC_THREADS) {
        const int2 q = parts[i];
        better(u32_as_f32((uint32_t)q.x), q.y, best, idx);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        better(ov, oi, best, idx);
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < DEC_THREADS / 64; w++) better(bv[w], bi[w], best, idx);
        if (idx == 0x7fffffff) idx = 0;
        *d_tok = idx;
        if (hist && pos >= 0 && pos < hist_len) hist[pos] = idx;
        *d_pos = pos + 1;
        tok = idx;
    }
    __syncthreads();
    const int64_t t = tok;
    const bool ok = t >= 0 && t < vocab;
    const float4 *src = (const float4 *)(table + (ok ? t : 0) * (int64_t)hidden);
    for (int i = threadIdx.x; i < hidden / 4; i += DEC_THREADS)
        ((float4 *)xout)[i] = ok ? src[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// The first maximum of each range of len values of x (a NaN never wins):
// workgroup b takes [b len, min(n, (b + 1) len)) and writes (bits of the
// value, index) to parts[b], the pairs argmax_parts_embed_kernel reduces.  For
// heads whose matvec does not keep the pairs itself.
__global__ __launch_bounds__(DEC_THREADS) void argmax_parts_kernel(const float *__restrict__ x, int n, int len,
                                                                   int2 *__restrict__ parts) {
    __shared__ float bv[DEC_THREADS / 64];
    __shared__ int bi[DEC_THREADS / 64];
    const int b0 = (int)blockIdx.x * len, b1 = min(n, b0 + len);
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = b0 + (int)threadIdx.x; i < b1; i += DEC_THREADS) better(x[i], i, best, idx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        better(ov, oi, best, idx);
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < DEC_THREADS / 64; w++) better(bv[w], bi[w], best, idx);
        parts[blockIdx.x] = make_int2((int)f32_as_u32(best), idx);
    }
}

}  // namespace

hipError_t launch_argmax_parts(const float *x, int64_t n, int2 *parts, int max_parts, int *nparts, hipStream_t s) {
    constexpr int LEN = 2 * DEC_THREADS;  // values per workgroup
    if (!x || !parts || !nparts || n <= 0 || n > 0x7fffffff) return hipErrorInvalidValue;
    const int64_t g = (n + LEN - 1) / LEN;
    if (g > max_parts) return hipErrorNotSupported;
    argmax_parts_kernel<<<(unsigned)g, DEC_THREADS, 0, s>>>(x, (int)n, LEN, parts);
    *nparts = (int)g;
    return hipGetLastError();
}

hipError_t launch_argmax_parts_embed(const int2 *parts, int nparts, int64_t *d_tok, int64_t *d_pos, int64_t *hist,
                                     int64_t hist_len, const float *table, int64_t vocab, int64_t hidden, float *xout,
                                     hipStream_t s) {
    if (!parts || nparts <= 0 || !d_tok || !d_pos || !table || !xout || vocab <= 0 || hidden <= 0 || hidden % 4 ||
        hidden > 0x7fffffff || (((uintptr_t)table | (uintptr_t)xout) & 15))
        return hipErrorInvalidValue;
    argmax_parts_embed_kernel<<<1, DEC_THREADS, 0, s>>>(parts, nparts, d_tok, d_pos, hist, hist_len, table, vocab,
                                                        (int)hidden, xout);
    return hipGetLastError();
}

hipError_t launch_embed(const float *table, int64_t vocab, const int64_t *d_tok, int64_t m, int64_t hidden, float *out,
                        hipStream_t s) {
    if (!table || !d_tok || !out || vocab <= 0 || hidden <= 0 || hidden % 4 || hidden > 0x7fffffff || m <= 0 ||
        m > 0x7fffffff || (((uintptr_t)table | (uintptr_t)out) & 15))
        return hipErrorInvalidValue;
    embed_kernel<<<(unsigned)m, DEC_THREADS, 0, s>>>(table, vocab, d_tok, (int)hidden, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(float *x, const float *delta, const float *w, int64_t m, int64_t n, float eps, float *out,
                          hipStream_t s) {
    if (!x || !w || !out || m <= 0 || n <= 0 || n % 4 || n > 4 * RMS_V * DEC_THREADS || m > 0x7fffffff)
        return hipErrorInvalidValue;
    rmsnorm_kernel<<<(unsigned)m, DEC_THREADS, 0, s>>>(x, delta, w, (int)n, eps, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_act(float *x, const float *delta, const float *w, int64_t m, int64_t n, float eps,
                              float *out, const ActPlanes &a, hipStream_t s) {
    if (!x || !w || !a.qs || !a.d || !a.bsums || !a.bsum16 || m <= 0 || n <= 0 || n % QK_K ||
        n > 4 * RMS_V * DEC_THREADS || m > 0x7fffffff)
        return hipErrorInvalidValue;
    rmsnorm_act_kernel<<<(unsigned)m, DEC_THREADS, 0, s>>>(x, delta, w, (int)n, eps, out, a);
    return hipGetLastError();
}

hipError_t launch_swiglu_pairs_act(const float *y, int64_t ld, int64_t m, int64_t n, float *out, const ActPlanes &a,
                                   hipStream_t s) {
    if (!y || !a.qs || !a.d || !a.bsums || !a.bsum16 || n <= 0 || n % QK_K || n > 0x7fffffff / 2 || m <= 0 ||
        m > 65535 || ld % 4 || (m > 1 && ld < 2 * n) || (((uintptr_t)y | (uintptr_t)out) & 15))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n / QK_K + DEC_THREADS / 64 - 1) / (DEC_THREADS / 64)), (unsigned)m);
    swiglu_pairs_act_kernel<<<grid, DEC_THREADS, 0, s>>>(y, ld, (int)n, out, a);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *g, const float *u, int64_t ld, int64_t m, int64_t n, float *out, hipStream_t s) {
    if (!g || !u || !out || n <= 0 || m <= 0 || m > 65535 || (m > 1 && ld < n)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n + DEC_THREADS - 1) / DEC_THREADS), (unsigned)m);
    silu_mul_kernel<<<grid, DEC_THREADS, 0, s>>>(g, u, ld, n, out);
    return hipGetLastError();
}

hipError_t launch_swiglu_pairs(const float *y, int64_t ld, int64_t m, int64_t n, float *out, hipStream_t s) {
    if (!y || !out || n <= 0 || n % 4 || m <= 0 || m > 65535 || (m > 1 && ld < 2 * n)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n + DEC_THREADS - 1) / DEC_THREADS), (unsigned)m);
    swiglu_pairs_kernel<<<grid, DEC_THREADS, 0, s>>>(y, ld, n, out);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const float *qk, const float *v, const float *cosb, const float *sinb,
                              const int64_t *d_pos, float *kc, float *vc, int64_t n_head, int64_t n_kv, int64_t hd,
                              int64_t max_seq, float *out, hipStream_t s) {
    if (!qk || !v || !cosb || !sinb || !d_pos || !kc || !vc || !out) return hipErrorInvalidValue;
    // hd: a multiple of 8 whose quarter is a power of two (lanes per position), dividing the workgroup
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || hd < 8 || hd > ATT_MAX_HD || (hd / 4) & (hd / 4 - 1) || hd % 4 ||
        max_seq <= 0 || max_seq > ATT_MAX_SEQ)
        return hipErrorInvalidValue;
    const unsigned grid = (unsigned)n_head;
    switch (hd / 4) {
    case 2: attn_decode_kernel<2><<<grid, WIDE_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head, (int)n_kv, (int)max_seq, out); break;
    case 4: attn_decode_kernel<4><<<grid, WIDE_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head, (int)n_kv, (int)max_seq, out); break;
    case 8: attn_decode_kernel<8><<<grid, WIDE_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head, (int)n_kv, (int)max_seq, out); break;
    case 16: attn_decode_kernel<16><<<grid, WIDE_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head, (int)n_kv, (int)max_seq, out); break;
    case 32: attn_decode_kernel<32><<<grid, WIDE_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head, (int)n_kv, (int)max_seq, out); break;
    case 64: attn_decode_kernel<64><<<grid, WIDE_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head, (int)n_kv, (int)max_seq, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int64_t n, int64_t *d_tok, int64_t *d_pos, int64_t *hist, int64_t hist_len,
                         hipStream_t s) {
    if (!x || !d_tok || !d_pos || n <= 0 || ((uintptr_t)x & 15) || n > 0x7fffffff) return hipErrorInvalidValue;
    argmax_kernel<<<1, WIDE_THREADS, 0, s>>>(x, (int)n, d_tok, d_pos, hist, hist_len);
    return hipGetLastError();
}

}  // namespace aq
