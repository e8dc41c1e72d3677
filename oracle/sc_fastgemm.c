/*
 * Test infrastructure, CPU baseline only: never a parity checker and never
 * linked into the product library.
 *
 * The reference's flex conv (crates/burn_flex_gmm/src/lib.rs:242-375) is an
 * im2col gather followed by matrixmultiply::sgemm (Cargo.lock:6677-6680 pins
 * matrixmultiply 0.3.10, whose sgemm packs A into MR-row panels and B into
 * NR-column panels of a KC-deep block and runs an MR x NR register tile of
 * fused multiply-adds).  oracle/sc_oracle.c restates that path with every
 * product and sum separately rounded (-ffp-contract=off), which is what
 * parity needs but runs the GEMM at a naive loop's speed.  This file times
 * the same algorithm with a GEMM of the packed, register-blocked kind, built
 * in its own object with FMA contraction (oracle/Makefile), so that the CPU
 * baseline is not understated:
 *   gather : the same im2col [n_q, K*Cin_g] as orc_conv_flex_precomputed
 *   sgemm  : C[m,n] += A[m,k] B[k,n]; B packed once into KC x 16 panels,
 *            A packed per (MC x KC) block into 6-row panels, a 6 x 16 tile
 *            of 8-wide float vectors (12 accumulators) per micro-kernel call
 *            (the usual AVX2 + FMA shape); OpenMP over MC-row blocks for the
 *            all-cores figure.
 * Results agree with the separately rounded oracle to float rounding (the
 * sums are the same, in another association).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "sc_oracle_cfg.h"

typedef float v8 __attribute__((vector_size(32)));

enum { MR = 6, NR = 16, KC = 384, MC = 120 };

static int g_fast_threads = 1;

void orc_fast_set_num_threads(int n) { g_fast_threads = n > 0 ? n : 1; }

/* B [k, n] (row stride ldb) -> panels of NR columns: panel j holds
 * B[p, j*NR .. j*NR+NR) for p in [0, k), NR floats per p (zeros past n). */
static void pack_b(int64_t k, int64_t n, const float *B, int64_t ldb, float *Bp)
{
    const int64_t np = (n + NR - 1) / NR;
    for (int64_t j = 0; j < np; ++j) {
        float *dst = Bp + j * k * NR;
        const int64_t c0 = j * NR, cw = n - c0 < NR ? n - c0 : NR;
        for (int64_t p = 0; p < k; ++p) {
            const float *src = B + p * ldb + c0;
            int64_t c = 0;
            for (; c < cw; ++c) dst[p * NR + c] = src[c];
            for (; c < NR; ++c) dst[p * NR + c] = 0.f;
        }
    }
}

/* A rows [i0, i0+mc) x cols [p0, p0+kc) -> panels of MR rows, MR floats per p
 * (zeros past the last row). */
static void pack_a(int64_t mc, int64_t kc, const float *A, int64_t lda, float *Ap)
{
    for (int64_t i = 0; i < mc; i += MR) {
        float *dst = Ap + i * kc;
        const int64_t rw = mc - i < MR ? mc - i : MR;
        for (int64_t p = 0; p < kc; ++p) {
            int64_t r = 0;
            for (; r < rw; ++r) dst[p * MR + r] = A[(i + r) * lda + p];
            for (; r < MR; ++r) dst[p * MR + r] = 0.f;
        }
    }
}

/* acc (MR x NR) += Ap panel (kc x MR) * Bp panel (kc x NR), then added to C
 * (rows < mr, columns < nr). */
static void micro(int64_t kc, const float *Ap, const float *Bp, float *C, int64_t ldc, int64_t mr, int64_t nr)
{
    v8 acc[MR][2];
    for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = (v8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma GCC unroll 4
    for (int64_t p = 0; p < kc; ++p) {
        v8 b0, b1;
        memcpy(&b0, Bp + p * NR, sizeof(v8));
        memcpy(&b1, Bp + p * NR + 8, sizeof(v8));
        const float *a = Ap + p * MR;
        for (int r = 0; r < MR; ++r) {
            const v8 av = (v8){a[r], a[r], a[r], a[r], a[r], a[r], a[r], a[r]};
            acc[r][0] += av * b0;
            acc[r][1] += av * b1;
        }
    }
    for (int64_t r = 0; r < mr; ++r) {
        float t[NR];
        memcpy(t, &acc[r][0], sizeof(v8));
        memcpy(t + 8, &acc[r][1], sizeof(v8));
        for (int64_t c = 0; c < nr; ++c) C[r * ldc + c] += t[c];
    }
}

/* C[m, n] += A[m, k] @ B[k, n] (row-major, strides lda / ldb / ldc). */
static int fast_sgemm_acc(int64_t m, int64_t k, int64_t n, const float *A, int64_t lda, const float *B,
                          int64_t ldb, float *C, int64_t ldc)
{
    const int64_t np = (n + NR - 1) / NR;
    float *Bp = (float *)aligned_alloc(64, sizeof(float) * (size_t)(np * k * NR + 16));
    if (!Bp) return ORC_ERR_ALLOC;
    pack_b(k, n, B, ldb, Bp);
    const int64_t nblk = (m + MC - 1) / MC;
    int bad = 0;
#pragma omp parallel for num_threads(g_fast_threads) schedule(static) reduction(| : bad) if (g_fast_threads > 1)
    for (int64_t bi = 0; bi < nblk; ++bi) {
        float *Ap = (float *)aligned_alloc(64, sizeof(float) * (size_t)(MC * KC + 16));
        if (!Ap) {
            bad = 1;
            continue;
        }
        const int64_t i0 = bi * MC, mc = m - i0 < MC ? m - i0 : MC;
        for (int64_t p0 = 0; p0 < k; p0 += KC) {
            const int64_t kc = k - p0 < KC ? k - p0 : KC;
            pack_a(mc, kc, A + i0 * lda + p0, lda, Ap);
            for (int64_t j = 0; j < np; ++j) {
                const int64_t nr = n - j * NR < NR ? n - j * NR : NR;
                const float *bp = Bp + j * k * NR + p0 * NR;
                for (int64_t i = 0; i < mc; i += MR) {
                    const int64_t mr = mc - i < MR ? mc - i : MR;
                    micro(kc, Ap + i * kc, bp, C + (i0 + i) * ldc + j * NR, ldc, mr, nr);
                }
            }
        }
        free(Ap);
    }
    free(Bp);
    return bad ? ORC_ERR_ALLOC : ORC_OK;
}

/* orc_conv_flex_precomputed's algorithm (bias, per group the im2col gather,
 * out += im2col @ packed) with fast_sgemm_acc; packed = pack_flex_weight(w),
 * [groups][K*Cin_g][Cout_g].  The gather runs on the same thread count. */
int orc_conv_flex_fast(const orc_cfg *c, const float *packed, const float *bias, const float *input, int64_t n_in,
                       const int32_t *nbr, int64_t n_q, float *out)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    if (n_in < n_q) return ORC_ERR_SHAPE;
    if (n_q == 0) return ORC_OK;
    const int64_t K = orc_kernel_rows(c), cin = c->in_channels_per_group, n = c->out_channels_per_group,
                  kin = K * cin, C_in = c->in_channels, C_out = c->out_channels;
    for (int64_t r = 0; r < n_q; ++r) memcpy(&out[r * C_out], bias, sizeof(float) * (size_t)C_out);
    float *g_buf = (float *)malloc(sizeof(float) * (size_t)(n_q * kin));
    if (!g_buf) return ORC_ERR_ALLOC;
    int rc = ORC_OK;
    for (int64_t g = 0; g < c->groups && rc == ORC_OK; ++g) {
        int bad = 0;
#pragma omp parallel for num_threads(g_fast_threads) schedule(static) reduction(| : bad) if (g_fast_threads > 1)
        for (int64_t r = 0; r < n_q; ++r) {
            for (int64_t k = 0; k < K; ++k) {
                const int32_t s = nbr[r * K + k];
                float *dst = &g_buf[r * kin + k * cin];
                if (s == ORC_INVALID_NEIGHBOR || s < 0 || s >= n_in) {
                    if (s != ORC_INVALID_NEIGHBOR) bad = 1;
                    memset(dst, 0, sizeof(float) * (size_t)cin);
                    continue;
                }
                memcpy(dst, &input[(int64_t)s * C_in + g * cin], sizeof(float) * (size_t)cin);
            }
        }
        if (bad) rc = ORC_ERR_INDEX;
        if (rc == ORC_OK) rc = fast_sgemm_acc(n_q, kin, n, g_buf, kin, &packed[g * kin * n], n, &out[g * n], C_out);
    }
    free(g_buf);
    return rc;
}
