/*
 * The oracle's C restatement (oracle/selection.c) under AddressSanitizer + UndefinedBehaviorSanitizer.
 *
 * Every buffer is a heap block of exactly the size the function's contract gives, so a read or
 * write one element outside it is reported. The inputs cover the edge cases of each function:
 * partial last blocks, k at and above the frame size, ties, signed zeros, infinities and NaN,
 * probe chunking below and above 256 rows, key sets with every mode and flag and out-of-range
 * parameters. Light property checks (ranges, order, counts) run beside them.
 * Exit status 0 when every check holds; the sanitizers abort on the first finding.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint32_t oracle_fkey(uint32_t bits);
void oracle_block_pool(const uint16_t* x, int64_t row_stride, int F, int T, int nspec, int D, int block, float* out);
void oracle_block_scores(const float* q, const float* k, int NQ, int NK, int D, float* scores);
int oracle_frame_topk(const float* scores, int NQ, int F, int C, int k, int32_t* out);
int oracle_global_topk(const float* scores, int NQ, int NC, int k, int32_t* out);
int oracle_probe_chunk(int N);
void oracle_probe_mean(const float* q, int64_t row_stride, int N, int D, float* out);
void oracle_probe_scores(const float* qbar, const float* k, int64_t row_stride, int N, int D, float scale, float* out);
int oracle_keyset(const float* scores, int N, int T, int ns, int mode, int param, int start, int include,
                  int32_t* out);

static int failures = 0;
#define CHECK(c)                                                                   \
    do {                                                                           \
        if (!(c)) {                                                                \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            ++failures;                                                            \
        }                                                                          \
    } while (0)

static uint32_t rng = 12345u;
static uint32_t next_u32(void) {
    rng ^= rng << 13;
    rng ^= rng >> 17;
    rng ^= rng << 5;
    return rng;
}
static float next_f(void) { return (float)(next_u32() >> 8) / 16777216.0f * 2.0f - 1.0f; }

static void* exact(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) abort();
    return p;
}

static void check_pool(void) {
    const int shapes[][3] = {{2, 69, 5}, {3, 155, 5}, {1, 6, 5}, {2, 64, 0}, {1, 1374, 5}};
    for (unsigned s = 0; s < sizeof(shapes) / sizeof(shapes[0]); ++s) {
        const int F = shapes[s][0], T = shapes[s][1], ns = shapes[s][2], D = 64;
        const int P = T - ns, NBf = (P + 63) / 64;
        uint16_t* x = (uint16_t*)exact(sizeof(uint16_t) * (size_t)F * T * D);
        for (int64_t i = 0; i < (int64_t)F * T * D; ++i) x[i] = (uint16_t)(0x3F80u + (next_u32() & 0x7F));  /* [1, 2) */
        float* out = (float*)exact(sizeof(float) * (size_t)F * NBf * D);
        oracle_block_pool(x, D, F, T, ns, D, 64, out);
        for (int64_t i = 0; i < (int64_t)F * NBf * D; ++i) CHECK(out[i] >= 1.0f && out[i] < 2.0f);
        free(x);
        free(out);
    }
}

static void check_scores_and_topk(void) {
    const int NQ = 5, F = 3, C = 7, D = 64;
    float* q = (float*)exact(sizeof(float) * NQ * D);
    float* k = (float*)exact(sizeof(float) * F * C * D);
    for (int i = 0; i < NQ * D; ++i) q[i] = next_f();
    for (int i = 0; i < F * C * D; ++i) k[i] = next_f();
    float* sc = (float*)exact(sizeof(float) * NQ * F * C);
    oracle_block_scores(q, k, NQ, F * C, D, sc);
    /* specials and ties in row 0 */
    sc[0] = -0.0f;
    sc[1] = 0.0f;
    sc[2] = INFINITY;
    sc[3] = -INFINITY;
    sc[4] = NAN;
    sc[5] = 0.0f;
    sc[6] = -1.0f;
    sc[C] = sc[C + 1] = sc[C + 2] = 1.0f;
    for (int c = 3; c < C; ++c) sc[C + c] = -1.0f;
    for (int kk = 1; kk <= C + 2; ++kk) {
        const int ke = kk < C ? kk : C;
        int32_t* out = (int32_t*)exact(sizeof(int32_t) * NQ * F * ke);
        CHECK(oracle_frame_topk(sc, NQ, F, C, kk, out) == 0);
        for (int i = 0; i < NQ; ++i)
            for (int f = 0; f < F; ++f)
                for (int t = 0; t < ke; ++t) {
                    const int32_t v = out[(i * F + f) * ke + t];
                    CHECK(v >= f * C && v < (f + 1) * C);
                }
        /* row 0 frame 0: +NaN sorts above +inf, +0 above -0, ties keep the lower index */
        if (ke >= 3) CHECK(out[0] == 4 && out[1] == 2 && out[2] == 1);
        if (ke >= 3) CHECK(out[ke] == C && out[ke + 1] == C + 1 && out[ke + 2] == C + 2);
        free(out);
        const int kg = kk < F * C ? kk : F * C;
        int32_t* g = (int32_t*)exact(sizeof(int32_t) * NQ * kg);
        CHECK(oracle_global_topk(sc, NQ, F * C, kk, g) == 0);
        for (int i = 0; i < NQ * kg; ++i) CHECK(g[i] >= 0 && g[i] < F * C);
        free(g);
    }
    CHECK(oracle_frame_topk(sc, NQ, F, C, 0, NULL) == -1);
    CHECK(oracle_frame_topk(sc, NQ, F, 0, 4, NULL) == -1);
    CHECK(oracle_global_topk(sc, NQ, 0, 4, NULL) == -1);
    CHECK(oracle_frame_topk(sc, NQ, F, 2000, 1500, NULL) == -2);
    CHECK(oracle_fkey(0x80000000u) < oracle_fkey(0x00000000u));
    free(q);
    free(k);
    free(sc);
}

static void check_probe(void) {
    const int Ns[] = {1, 255, 256, 257, 1000};
    for (unsigned s = 0; s < sizeof(Ns) / sizeof(Ns[0]); ++s) {
        const int N = Ns[s], D = 64;
        const int64_t stride = 80; /* rows wider than D */
        float* q = (float*)exact(sizeof(float) * (size_t)((N - 1) * stride + D));
        for (int64_t i = 0; i < (N - 1) * stride + D; ++i) q[i] = next_f();
        float* qbar = (float*)exact(sizeof(float) * D);
        oracle_probe_mean(q, stride, N, D, qbar);
        for (int d = 0; d < D; ++d) CHECK(fabsf(qbar[d]) <= 1.0f);
        float* sc = (float*)exact(sizeof(float) * N);
        oracle_probe_scores(qbar, q, stride, N, D, 0.125f, sc);
        for (int t = 0; t < N; ++t) CHECK(isfinite(sc[t]));
        CHECK(oracle_probe_chunk(N) * 256 >= N);
        free(q);
        free(qbar);
        free(sc);
    }
}

static void check_keyset(void) {
    const int T = 13, ns = 3, F = 4, N = F * T;
    float* sc = (float*)exact(sizeof(float) * N);
    for (int t = 0; t < N; ++t) sc[t] = (float)(next_u32() % 5); /* many ties */
    sc[7] = NAN;
    const int params[] = {1, 2, 5, N - 1, N, N + 10};
    for (int mode = 0; mode < 2; ++mode)
        for (unsigned pi = 0; pi < sizeof(params) / sizeof(params[0]); ++pi)
            for (int start = 0; start < 3; ++start)
                for (int inc = 0; inc < 2; ++inc) {
                    int32_t* out = (int32_t*)exact(sizeof(int32_t) * N);
                    const int n = oracle_keyset(sc, N, T, ns, mode, params[pi], start, inc, out);
                    CHECK(n >= 0 && n <= N);
                    for (int i = 1; i < n; ++i) CHECK(out[i] > out[i - 1]);
                    for (int i = 0; i < n; ++i) CHECK(out[i] >= 0 && out[i] < N);
                    if (mode == 1) {
                        const int want = params[pi] < N ? params[pi] : N;
                        CHECK(n >= want);
                    }
                    free(out);
                }
    /* rejected parameters: nothing written */
    CHECK(oracle_keyset(sc, N, T, ns, 0, 0, 0, 0, NULL) == -1);
    CHECK(oracle_keyset(sc, N, T, ns, 0, 3, -1, 0, NULL) == -1);
    CHECK(oracle_keyset(sc, N, T, ns, 2, 3, 0, 0, NULL) == -1);
    CHECK(oracle_keyset(sc, 0, T, ns, 0, 3, 0, 0, NULL) == -1);
    /* a start past the end selects nothing but the include set */
    int32_t* out = (int32_t*)exact(sizeof(int32_t) * N);
    CHECK(oracle_keyset(sc, N, T, ns, 0, 3, N + 5, 0, out) == 0);
    CHECK(oracle_keyset(sc, N, T, ns, 0, 3, N + 5, 1, out) == T + (F - 1) * ns);
    free(out);
    free(sc);
}

int main(void) {
    check_pool();
    check_scores_and_topk();
    check_probe();
    check_keyset();
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("oracle checks passed\n");
    return 0;
}
