/*
 * aq_capi_check.c -- the C ABI of libarm_ai_amd.so (include/aq.h) called
 * from compiled C, as the Rust NIF crate's `extern "C"` binding calls it,
 * checked against the CPU oracle (oracle/oracle.h, the restatement of
 * candle-core 0.8.4's k_quants).  Built by tests/c/Makefile with gcc; run by
 * tests/test_c_abi_program.py on a GPU box.  Test infrastructure: it links
 * the oracle as the checker.
 *
 * Checks, for Q4_K, Q6_K and Q8_0 weights built from seeded random bytes
 * (valid f16 scales), at m = 1 (matvec), 3 (batched matvec) and 40 (prefill
 * GEMM):
 *   - aq_qmatmul_f32 against orc_matmul within 1e-5 of the largest |value|;
 *   - aq_qmatmul_block_sums against orc_block_sums, bit for bit;
 *   - aq_quantize_q8k / aq_quantize_q8_0 against the oracle's quantizers,
 *     byte for byte;
 *   - the error paths a caller maps to candle's errors: k that is not the
 *     weight's k, a byte count that does not match the shape, a null
 *     pointer -- each a negative status with a message, never a crash.
 * Prints one line per check and "ALL OK" at the end; exit status 0 only
 * then.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "aq.h"
#include "oracle.h"

static int failures = 0;

#define CHECK(cond, ...)                      \
    do {                                      \
        if (!(cond)) {                        \
            printf("FAIL: " __VA_ARGS__);     \
            printf("\n");                     \
            failures++;                       \
        }                                     \
    } while (0)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (uint32_t)(rng_state >> 16);
}
static float rndf(void) { return (float)((double)rnd() / 4294967296.0 * 2.0 - 1.0); }

/* Random blocks of one type with finite, modest f16 scales at the spec's offsets. */
static uint8_t *make_weight(int type, int64_t n, int64_t k, size_t *nbytes) {
    const size_t bb = orc_type_block_bytes(type);
    const int64_t be = orc_type_block_elems(type);
    const size_t nblk = (size_t)(n * (k / be));
    uint8_t *w = malloc(nblk * bb);
    for (size_t i = 0; i < nblk * bb; i++) w[i] = (uint8_t)rnd();
    for (size_t b = 0; b < nblk; b++) {
        uint8_t *blk = w + b * bb;
        const uint16_t d = orc_f32_to_f16(0.002f + 0.01f * (float)(rnd() % 1000) / 1000.0f);
        const uint16_t dmin = orc_f32_to_f16(0.001f + 0.005f * (float)(rnd() % 1000) / 1000.0f);
        if (type == ORC_Q4_K) {
            memcpy(blk, &d, 2);
            memcpy(blk + 2, &dmin, 2);
        } else if (type == ORC_Q6_K) {
            memcpy(blk + 208, &d, 2);
        } else if (type == ORC_Q8_0) {
            memcpy(blk, &d, 2);
        }
    }
    *nbytes = nblk * bb;
    return w;
}

static double rel_err(const float *a, const float *b, size_t n) {
    double num = 0.0, den = 1e-30;
    for (size_t i = 0; i < n; i++) {
        const double d = fabs((double)a[i] - (double)b[i]);
        if (d > num) num = d;
        if (fabs((double)b[i]) > den) den = fabs((double)b[i]);
    }
    return num / den;
}

static void check_weight(aq_ctx *ctx, int type, const char *name, int64_t n, int64_t k) {
    size_t nbytes = 0;
    uint8_t *wb = make_weight(type, n, k, &nbytes);
    aq_qweight *w = NULL;
    int rc = aq_qweight_upload(ctx, type, wb, nbytes, n, k, &w);
    CHECK(rc == AQ_OK, "%s upload: %d %s", name, rc, aq_last_error());
    if (rc != AQ_OK) {
        free(wb);
        return;
    }
    int t = 0;
    int64_t qn = 0, qk = 0;
    size_t dev = 0;
    rc = aq_qweight_info(w, &t, &qn, &qk, &dev);
    CHECK(rc == AQ_OK && t == type && qn == n && qk == k && dev >= nbytes, "%s info", name);

    const int ms[3] = {1, 3, 40};
    for (int mi = 0; mi < 3; mi++) {
        const int64_t m = ms[mi];
        float *x = malloc(sizeof(float) * m * k);
        for (int64_t i = 0; i < m * k; i++) x[i] = rndf() * (i % 97 == 0 ? 8.0f : 1.0f);
        float *y = malloc(sizeof(float) * m * n), *yr = malloc(sizeof(float) * m * n);
        rc = aq_qmatmul_f32(ctx, w, x, m, k, y);
        CHECK(rc == AQ_OK, "%s m=%lld matmul: %d %s", name, (long long)m, rc, aq_last_error());
        CHECK(orc_matmul(type, m, k, n, x, wb, yr, 0) == 0, "%s oracle matmul", name);
        const double e = rel_err(y, yr, (size_t)(m * n));
        CHECK(e <= 1e-5, "%s m=%lld: rel %.3e", name, (long long)m, e);
        printf("%s %lldx%lld m=%lld: aq_qmatmul_f32 rel %.2e vs the oracle\n", name, (long long)n, (long long)k,
               (long long)m, e);

        /* integer block sums, bit for bit (m = 1 and 3: the matvec; 40: the GEMM epilogue) */
        const int64_t be = orc_type_block_elems(type), nblk = k / be;
        int32_t *S = malloc(sizeof(int32_t) * m * n * nblk), *Sm = malloc(sizeof(int32_t) * m * n * nblk);
        int32_t *So = malloc(sizeof(int32_t) * m * n * nblk), *Smo = malloc(sizeof(int32_t) * m * n * nblk);
        rc = aq_qmatmul_block_sums(ctx, w, x, m, k, S, Sm);
        CHECK(rc == AQ_OK, "%s block sums: %d %s", name, rc, aq_last_error());
        const int act = type == ORC_Q8_0 ? ORC_Q8_0 : ORC_Q8_K;
        const size_t ab = orc_type_block_bytes(act) * (size_t)(k / orc_type_block_elems(act));
        uint8_t *xq = malloc(ab * (size_t)m);
        for (int64_t r = 0; r < m; r++) {
            if (act == ORC_Q8_K) orc_quantize_row_q8k(x + r * k, k, xq + r * ab);
            else orc_quantize_row_q8_0(x + r * k, k, xq + r * ab);
        }
        orc_block_sums_mat(type, m, n, k, wb, xq, So, Smo, 0);
        int same = memcmp(S, So, sizeof(int32_t) * m * n * nblk) == 0;
        if (type == ORC_Q4_K) same = same && memcmp(Sm, Smo, sizeof(int32_t) * m * n * nblk) == 0;
        CHECK(same, "%s m=%lld: integer block sums differ from the oracle", name, (long long)m);
        printf("%s m=%lld: block sums %s\n", name, (long long)m, same ? "bit-exact" : "DIFFER");

        /* the activation quantizer the matmul used, byte for byte */
        uint8_t *gq = malloc(ab * (size_t)m);
        rc = act == ORC_Q8_K ? aq_quantize_q8k(ctx, x, m, k, gq) : aq_quantize_q8_0(ctx, x, m, k, gq);
        CHECK(rc == AQ_OK && memcmp(gq, xq, ab * (size_t)m) == 0, "%s m=%lld: quantised activation differs", name,
              (long long)m);
        free(gq);
        free(xq);
        free(S);
        free(Sm);
        free(So);
        free(Smo);
        free(x);
        free(y);
        free(yr);
    }

    /* error paths */
    float xs[512] = {0}, ys[8];
    rc = aq_qmatmul_f32(ctx, w, xs, 1, k + 256, ys);
    CHECK(rc == AQ_ERR_SHAPE && strlen(aq_last_error()) > 0, "%s: wrong k gives %d", name, rc);
    rc = aq_qmatmul_f32(ctx, w, NULL, 1, k, ys);
    CHECK(rc == AQ_ERR_INVALID_ARG, "%s: null lhs gives %d", name, rc);
    aq_qweight *w2 = NULL;
    rc = aq_qweight_upload(ctx, type, wb, nbytes - 1, n, k, &w2);
    CHECK(rc == AQ_ERR_SHAPE && w2 == NULL, "%s: short byte count gives %d", name, rc);
    CHECK(aq_qweight_free(w) == AQ_OK, "%s free", name);
    free(wb);
}

int main(void) {
    printf("aq_abi_version %d\n", aq_abi_version());
    CHECK(aq_abi_version() == 1, "abi version");
    int ndev = 0;
    CHECK(aq_device_count(&ndev) == AQ_OK && ndev >= 1, "no device (%d)", ndev);
    if (ndev < 1) return 1;
    aq_ctx *ctx = NULL;
    int rc = aq_ctx_create(0, &ctx);
    CHECK(rc == AQ_OK && ctx, "ctx create: %d %s", rc, aq_last_error());
    if (!ctx) return 1;
    check_weight(ctx, ORC_Q4_K, "Q4_K", 1000, 2048);
    check_weight(ctx, ORC_Q6_K, "Q6_K", 600, 1536);
    check_weight(ctx, ORC_Q8_0, "Q8_0", 520, 1024);
    CHECK(aq_ctx_destroy(ctx) == AQ_OK, "ctx destroy");
    if (failures) {
        printf("%d FAILED\n", failures);
        return 1;
    }
    printf("ALL OK\n");
    return 0;
}
