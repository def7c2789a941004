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

constexpr int DEC_THREADS = 256;

// sum over a 256-thread block; every thread gets the result.  red: >= 4 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// out[row] = embedding row *d_tok (a token id outside [0, vocab) gives zeros).
__global__ __launch_bounds__(DEC_THREADS) void embed_kernel(const float *__restrict__ table, int64_t vocab,
                                                            const int64_t *__restrict__ d_tok, int hidden,
                                                            float *__restrict__ out) {
    const int64_t t = *d_tok;
    const bool ok = t >= 0 && t < vocab;
    for (int i = threadIdx.x; i < hidden; i += DEC_THREADS) out[i] = ok ? table[t * hidden + i] : 0.0f;
}

// One row per workgroup: x += delta (when delta is given, written back to x:
// the residual stream), then out = x / sqrt(sum(x^2)/n + eps) * w.
__global__ __launch_bounds__(DEC_THREADS) void rmsnorm_kernel(float *__restrict__ x, const float *__restrict__ delta,
                                                              const float *__restrict__ w, int n, float eps,
                                                              float *__restrict__ out) {
    __shared__ float red[4];
    float *xr = x + (int64_t)blockIdx.x * n;
    const float *dr = delta ? delta + (int64_t)blockIdx.x * n : nullptr;
    float *orow = out + (int64_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += DEC_THREADS) {
        float v = xr[i];
        if (dr) {
            v += dr[i];
            xr[i] = v;
        }
        ss = __builtin_fmaf(v, v, ss);
    }
    const float m = sqrtf(block_sum(ss, red) / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += DEC_THREADS) orow[i] = (xr[i] / m) * w[i];
}

// out = silu(g) * u.  gu = [g (n) | u (n)] per row (the merged w1|w3 output).
__global__ __launch_bounds__(DEC_THREADS) void silu_mul_kernel(const float *__restrict__ gu, int64_t n,
                                                               float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * DEC_THREADS + threadIdx.x;
    if (i >= n) return;
    const float g = gu[i];
    out[i] = (g / (1.0f + expf(-g))) * gu[n + i];
}

// Attention for one query position at *d_pos, one workgroup per query head.
// qk = [q (n_head*hd) | k (n_kv*hd)] before rotation, v (n_kv*hd); the
// caches are [n_kv][max_seq][hd] for this layer.  Each workgroup rotates its
// q head and its group's k (rope_i: pairs (2i, 2i+1) by pos * theta_i, from
// the cos/sin tables [max_seq][hd/2]); the first workgroup of each group
// stores the rotated k and v at pos for later steps, and every workgroup uses
// its own registers for position pos, so no workgroup waits for another.
constexpr int ATT_MAX_SEQ = 8192;
constexpr int ATT_MAX_HD = 256;
__global__ __launch_bounds__(DEC_THREADS) void attn_decode_kernel(
    const float *__restrict__ qk, const float *__restrict__ v, const float *__restrict__ cosb,
    const float *__restrict__ sinb, const int64_t *__restrict__ d_pos, float *__restrict__ kc, float *__restrict__ vc,
    int n_head, int n_kv, int hd, int max_seq, float *__restrict__ out) {
    __shared__ float qs[ATT_MAX_HD], ks[ATT_MAX_HD], vs[ATT_MAX_HD];
    __shared__ float sc[ATT_MAX_SEQ];
    __shared__ float red[4];
    __shared__ float part[DEC_THREADS];
    const int head = blockIdx.x, tid = threadIdx.x;
    const int rep = n_head / n_kv, kvh = head / rep;
    const int64_t pos = *d_pos;
    if (pos < 0 || pos >= max_seq) return;  // the host checks; never index out of the cache
    const float *q0 = qk + (int64_t)head * hd;
    const float *k0 = qk + (int64_t)n_head * hd + (int64_t)kvh * hd;
    const float *v0 = v + (int64_t)kvh * hd;
    const float *cr = cosb + pos * (hd / 2), *sr = sinb + pos * (hd / 2);
    for (int i = tid; i < hd / 2; i += DEC_THREADS) {
        const float c = cr[i], s = sr[i];
        const float a = q0[2 * i], b = q0[2 * i + 1];
        qs[2 * i] = a * c - b * s;
        qs[2 * i + 1] = a * s + b * c;
        const float ka = k0[2 * i], kb = k0[2 * i + 1];
        ks[2 * i] = ka * c - kb * s;
        ks[2 * i + 1] = ka * s + kb * c;
    }
    for (int i = tid; i < hd; i += DEC_THREADS) vs[i] = v0[i];
    __syncthreads();
    float *kh = kc + (int64_t)kvh * max_seq * hd;
    float *vh = vc + (int64_t)kvh * max_seq * hd;
    if (head % rep == 0)
        for (int i = tid; i < hd; i += DEC_THREADS) {
            kh[pos * hd + i] = ks[i];
            vh[pos * hd + i] = vs[i];
        }
    // scores q . k_p / sqrt(hd) for p = 0..pos (k_pos from LDS)
    const float rs = sqrtf((float)hd);
    float mx = -INFINITY;
    for (int64_t p = tid; p <= pos; p += DEC_THREADS) {
        const float *kp = p == pos ? ks : kh + p * hd;
        float d = 0.0f;
        for (int i = 0; i < hd; i += 4) {
            const float4 kv4 = *(const float4 *)(kp + i);
            d = __builtin_fmaf(qs[i], kv4.x, d);
            d = __builtin_fmaf(qs[i + 1], kv4.y, d);
            d = __builtin_fmaf(qs[i + 2], kv4.z, d);
            d = __builtin_fmaf(qs[i + 3], kv4.w, d);
        }
        const float s = d / rs;
        sc[p] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);
    float sum = 0.0f;
    for (int64_t p = tid; p <= pos; p += DEC_THREADS) {
        const float e = expf(sc[p] - mx);
        sc[p] = e;
        sum += e;
    }
    sum = block_sum(sum, red);  // its barriers also publish sc[]
    // out[d] = sum_p (e_p / sum) v_p[d]: thread (d, g) takes positions p = g mod groups
    const int groups = DEC_THREADS / hd;
    const int d = tid % hd, g = tid / hd;
    float acc = 0.0f;
    if (g < groups)
        for (int64_t p = g; p <= pos; p += groups) {
            const float vv = p == pos ? vs[d] : vh[p * hd + d];
            acc = __builtin_fmaf(sc[p] / sum, vv, acc);
        }
    part[tid] = acc;
    __syncthreads();
    if (tid < hd) {
        float o = 0.0f;
        for (int j = 0; j < groups; j++) o += part[j * hd + tid];
        out[(int64_t)head * hd + tid] = o;
    }
}

// Greedy pick: the first index of the largest value (a NaN never wins; all
// NaN gives 0).  Writes it to *d_tok (the next step's input), to
// hist[*d_pos] when hist is given, and advances *d_pos by one.
__global__ __launch_bounds__(DEC_THREADS) void argmax_kernel(const float *__restrict__ x, int n,
                                                             int64_t *__restrict__ d_tok, int64_t *__restrict__ d_pos,
                                                             int64_t *__restrict__ hist, int64_t hist_len) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += DEC_THREADS) {
        const float v = x[i];
        if (v > best || (v == best && i < idx)) {  // NaN compares false
            best = v;
            idx = i;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        if (idx == 0x7fffffff) idx = 0;
        const int64_t pos = *d_pos;
        *d_tok = idx;
        if (hist && pos >= 0 && pos < hist_len) hist[pos] = idx;
        *d_pos = pos + 1;
    }
}

}  // namespace

hipError_t launch_embed(const float *table, int64_t vocab, const int64_t *d_tok, int64_t hidden, float *out,
                        hipStream_t s) {
    if (!table || !d_tok || !out || vocab <= 0 || hidden <= 0 || hidden > 0x7fffffff) return hipErrorInvalidValue;
    embed_kernel<<<1, DEC_THREADS, 0, s>>>(table, vocab, d_tok, (int)hidden, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(float *x, const float *delta, const float *w, int64_t m, int64_t n, float eps, float *out,
                          hipStream_t s) {
    if (!x || !w || !out || m <= 0 || n <= 0 || n > 0x7fffffff || m > 0x7fffffff) return hipErrorInvalidValue;
    rmsnorm_kernel<<<(unsigned)m, DEC_THREADS, 0, s>>>(x, delta, w, (int)n, eps, out);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *gu, int64_t n, float *out, hipStream_t s) {
    if (!gu || !out || n <= 0) return hipErrorInvalidValue;
    silu_mul_kernel<<<(unsigned)((n + DEC_THREADS - 1) / DEC_THREADS), DEC_THREADS, 0, s>>>(gu, n, out);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const float *qk, const float *v, const float *cosb, const float *sinb,
                              const int64_t *d_pos, float *kc, float *vc, int64_t n_head, int64_t n_kv, int64_t hd,
                              int64_t max_seq, float *out, hipStream_t s) {
    if (!qk || !v || !cosb || !sinb || !d_pos || !kc || !vc || !out) return hipErrorInvalidValue;
    if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || hd <= 0 || hd % 4 || hd > ATT_MAX_HD || DEC_THREADS % hd ||
        max_seq <= 0 || max_seq > ATT_MAX_SEQ)
        return hipErrorInvalidValue;
    attn_decode_kernel<<<(unsigned)n_head, DEC_THREADS, 0, s>>>(qk, v, cosb, sinb, d_pos, kc, vc, (int)n_head,
                                                                (int)n_kv, (int)hd, (int)max_seq, out);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int64_t n, int64_t *d_tok, int64_t *d_pos, int64_t *hist, int64_t hist_len,
                         hipStream_t s) {
    if (!x || !d_tok || !d_pos || n <= 0 || n > 0x7fffffff) return hipErrorInvalidValue;
    argmax_kernel<<<1, DEC_THREADS, 0, s>>>(x, (int)n, d_tok, d_pos, hist, hist_len);
    return hipGetLastError();
}

}  // namespace aq
