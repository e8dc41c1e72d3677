/*
 * sc_oracle.c -- CPU restatement of the reference's sparse-conv path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP product in
 * bevy_synth_amd/; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  Nothing in the product links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the mosure/bevy_synth repository root).  The reference is Rust (burn_flex_gmm
 * + burn_trellis) and cannot be compiled in this image (no cargo), so the
 * restatement is pinned by the reference's own known-answer tests, by two
 * independent formulations that must agree (flex gather+GEMM vs legacy direct
 * loop; hash build vs brute-force scan), and by closed forms -- see
 * tests/test_oracle.py.
 *
 * Build: oracle/Makefile  ->  oracle/liboracle.so
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "sc_oracle_cfg.h"

/* validate_config, crates/burn_flex_gmm/src/lib.rs:698-725. */
int orc_validate_config(const orc_cfg *c)
{
    if (c->in_channels <= 0 || c->out_channels <= 0) return ORC_ERR_CONFIG;
    if (c->kernel_d <= 0 || c->kernel_h <= 0 || c->kernel_w <= 0) return ORC_ERR_CONFIG;
    if (c->groups <= 0) return ORC_ERR_CONFIG;
    if (c->in_channels_per_group * c->groups != c->in_channels) return ORC_ERR_CONFIG;
    if (c->out_channels_per_group * c->groups != c->out_channels) return ORC_ERR_CONFIG;
    int used[3] = {0, 0, 0};
    for (int j = 0; j < 3; ++j) {
        int a = c->axis_order[j];
        if (a < 0 || a > 2 || used[a]) return ORC_ERR_CONFIG;
        used[a] = 1;
    }
    return ORC_OK;
}

/* kernel_rows, crates/burn_flex_gmm/src/lib.rs:59-67. */
int64_t orc_kernel_rows(const orc_cfg *c)
{
    if (orc_validate_config(c) != ORC_OK) return -1;
    return c->kernel_d * c->kernel_h * c->kernel_w;
}

/*
 * kernel_layout, crates/burn_flex_gmm/src/lib.rs:727-752 (identical to
 * kernel_offsets, crates/burn_flex_gmm/src/wgpu/neighbor.rs:190-217):
 * k = (kd*KH + kh)*KW + kw; delta_j = sign_j*(idx_j - floor(dim_j/2)) is
 * written to spatial axis axis_order[j].  offsets is [K][3] (x,y,z).
 */
int64_t orc_kernel_layout(const orc_cfg *c, int32_t *offsets)
{
    if (orc_validate_config(c) != ORC_OK) return -1;
    int32_t cd = (int32_t)(c->kernel_d / 2), ch = (int32_t)(c->kernel_h / 2),
            cw = (int32_t)(c->kernel_w / 2);
    int64_t k = 0;
    for (int64_t kd = 0; kd < c->kernel_d; ++kd)
        for (int64_t kh = 0; kh < c->kernel_h; ++kh)
            for (int64_t kw = 0; kw < c->kernel_w; ++kw) {
                int32_t d[3] = {c->axis_sign[0] * ((int32_t)kd - cd),
                                c->axis_sign[1] * ((int32_t)kh - ch),
                                c->axis_sign[2] * ((int32_t)kw - cw)};
                int32_t o[3] = {0, 0, 0};
                o[c->axis_order[0]] = d[0];
                o[c->axis_order[1]] = d[1];
                o[c->axis_order[2]] = d[2];
                offsets[3 * k + 0] = o[0];
                offsets[3 * k + 1] = o[1];
                offsets[3 * k + 2] = o[2];
                ++k;
            }
    return k;
}

/* ---- a plain open-addressing map (batch,x,y,z) -> row, standing in for the
 *      std HashMap of crates/burn_flex_gmm/src/lib.rs:80-86 ---- */
typedef struct {
    uint32_t key[4];
    int64_t row;
    int used;
} orc_slot;

typedef struct {
    orc_slot *slots;
    uint64_t mask;
} orc_map;

static uint64_t orc_hash4(const uint32_t k[4])
{
    uint64_t h = 0x9e3779b97f4a7c15ull;
    for (int i = 0; i < 4; ++i) {
        h ^= (uint64_t)k[i] + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
        h *= 0xbf58476d1ce4e5b9ull;
        h ^= h >> 31;
    }
    return h;
}

static int orc_map_init(orc_map *m, int64_t n)
{
    uint64_t cap = 16;
    while (cap < (uint64_t)n * 2 + 16) cap <<= 1;
    m->slots = (orc_slot *)calloc(cap, sizeof(orc_slot));
    m->mask = cap - 1;
    return m->slots ? ORC_OK : ORC_ERR_ALLOC;
}

static void orc_map_free(orc_map *m) { free(m->slots); }

/* insert = HashMap::insert: a later row with the same coord overwrites. */
static void orc_map_insert_last(orc_map *m, const uint32_t k[4], int64_t row)
{
    uint64_t s = orc_hash4(k) & m->mask;
    for (;;) {
        orc_slot *sl = &m->slots[s];
        if (!sl->used) {
            memcpy(sl->key, k, sizeof(sl->key));
            sl->row = row;
            sl->used = 1;
            return;
        }
        if (memcmp(sl->key, k, sizeof(sl->key)) == 0) {
            sl->row = row;
            return;
        }
        s = (s + 1) & m->mask;
    }
}

/* keep the lowest row on duplicates (device semantics). */
static void orc_map_insert_first(orc_map *m, const uint32_t k[4], int64_t row)
{
    uint64_t s = orc_hash4(k) & m->mask;
    for (;;) {
        orc_slot *sl = &m->slots[s];
        if (!sl->used) {
            memcpy(sl->key, k, sizeof(sl->key));
            sl->row = row;
            sl->used = 1;
            return;
        }
        if (memcmp(sl->key, k, sizeof(sl->key)) == 0) return;
        s = (s + 1) & m->mask;
    }
}

static int64_t orc_map_get(const orc_map *m, const uint32_t k[4])
{
    uint64_t s = orc_hash4(k) & m->mask;
    for (;;) {
        const orc_slot *sl = &m->slots[s];
        if (!sl->used) return -1;
        if (memcmp(sl->key, k, sizeof(sl->key)) == 0) return sl->row;
        s = (s + 1) & m->mask;
    }
}

/*
 * build_neighbor_rows, crates/burn_flex_gmm/src/lib.rs:69-109.
 * coords: [n][4] u32 (batch,x,y,z).  out: [n][K] i32, -1 where absent.
 * lowest_row_on_duplicate = 0 reproduces the CPU HashMap (last duplicate
 * wins, :83-86); = 1 reproduces every device algorithm (lowest row,
 * crates/burn_flex_gmm/src/wgpu/neighbor_kernels.rs:30-40,249-256,419-422).
 * query_rows < n maps only the first query_rows coords against the full set.
 */
int orc_build_neighbor_rows(const orc_cfg *c, const uint32_t *coords, int64_t n,
                            int64_t query_rows, int lowest_row_on_duplicate, int32_t *out)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    if (n > INT32_MAX || query_rows > n || query_rows < 0) return ORC_ERR_SHAPE;
    if (n == 0) return ORC_OK;
    int64_t K = orc_kernel_rows(c);
    int32_t *off = (int32_t *)malloc(sizeof(int32_t) * 3 * (size_t)K);
    if (!off) return ORC_ERR_ALLOC;
    orc_kernel_layout(c, off);
    orc_map m;
    if (orc_map_init(&m, n) != ORC_OK) {
        free(off);
        return ORC_ERR_ALLOC;
    }
    for (int64_t r = 0; r < n; ++r) {
        if (lowest_row_on_duplicate)
            orc_map_insert_first(&m, &coords[4 * r], r);
        else
            orc_map_insert_last(&m, &coords[4 * r], r);
    }
    for (int64_t r = 0; r < query_rows; ++r) {
        const uint32_t *q = &coords[4 * r];
        int32_t ox = (int32_t)q[1], oy = (int32_t)q[2], oz = (int32_t)q[3];
        for (int64_t k = 0; k < K; ++k) {
            int32_t nx = ox + off[3 * k], ny = oy + off[3 * k + 1], nz = oz + off[3 * k + 2];
            int32_t v = ORC_INVALID_NEIGHBOR;
            if (!(nx < 0 || ny < 0 || nz < 0)) {
                uint32_t key[4] = {q[0], (uint32_t)nx, (uint32_t)ny, (uint32_t)nz};
                int64_t hit = orc_map_get(&m, key);
                if (hit >= 0) v = (int32_t)hit;
            }
            out[r * K + k] = v;
        }
    }
    orc_map_free(&m);
    free(off);
    return ORC_OK;
}

/*
 * Brute-force scan, the semantics of neighbor_rows_from_coords_kernel
 * (crates/burn_flex_gmm/src/wgpu/neighbor_kernels.rs:3-46): for each
 * (row,k) the FIRST row whose coord equals coord+offset[k]; -1 if any
 * component of the neighbour is negative.  O(n^2 K): tiny inputs only.
 */
int orc_build_neighbor_rows_scan(const orc_cfg *c, const uint32_t *coords, int64_t n,
                                 int32_t *out)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    int64_t K = orc_kernel_rows(c);
    int32_t *off = (int32_t *)malloc(sizeof(int32_t) * 3 * (size_t)(K ? K : 1));
    if (!off) return ORC_ERR_ALLOC;
    orc_kernel_layout(c, off);
    for (int64_t r = 0; r < n; ++r) {
        const int32_t *q = (const int32_t *)&coords[4 * r];
        for (int64_t k = 0; k < K; ++k) {
            int32_t nx = q[1] + off[3 * k], ny = q[2] + off[3 * k + 1], nz = q[3] + off[3 * k + 2];
            int32_t found = ORC_INVALID_NEIGHBOR;
            for (int64_t s = 0; s < n; ++s) {
                const int32_t *p = (const int32_t *)&coords[4 * s];
                if (p[0] == q[0] && p[1] == nx && p[2] == ny && p[3] == nz) {
                    found = (int32_t)s;
                    break;
                }
            }
            if (nx < 0 || ny < 0 || nz < 0) found = ORC_INVALID_NEIGHBOR;
            out[r * K + k] = found;
        }
    }
    free(off);
    return ORC_OK;
}

/*
 * pack_flex_weight, crates/burn_flex_gmm/src/lib.rs:377-426:
 * [Cout,KD,KH,KW,Cin_g] -> per group [K*Cin_g, Cout_g], k-major then input
 * channel.
 */
int orc_pack_flex_weight(const orc_cfg *c, const float *w, float *packed)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    int64_t K = orc_kernel_rows(c), cin = c->in_channels_per_group,
            n = c->out_channels_per_group, kin = K * cin;
    for (int64_t g = 0; g < c->groups; ++g)
        for (int64_t ol = 0; ol < n; ++ol) {
            int64_t o = g * n + ol;
            for (int64_t k = 0; k < K; ++k)
                for (int64_t i = 0; i < cin; ++i)
                    packed[g * kin * n + (k * cin + i) * n + ol] = w[(o * K + k) * cin + i];
        }
    return ORC_OK;
}

/* Threads of the flex conv's gather and sgemm (1: the reference's
 * single-threaded matrixmultiply; more: the all-cores CPU baseline, OpenMP
 * over 64-row blocks).  Each row is computed by one thread in the same
 * operation order, so results do not depend on the thread count. */
static int g_orc_threads = 1;

void orc_set_num_threads(int n) { g_orc_threads = n > 0 ? n : 1; }

/* C[m,n] += A[m,k] @ B[k,n], row-major.  Stands in for the
 * matrixmultiply::sgemm call at crates/burn_flex_gmm/src/lib.rs:354-371
 * (alpha=1, beta=1: the product is formed, then added to C). */
static void orc_sgemm_acc(int64_t m, int64_t k, int64_t n, const float *A, int64_t lda,
                          const float *B, int64_t ldb, float *C, int64_t ldc)
{
    const int64_t MB = 64, KB = 256;
    const int64_t nblk = (m + MB - 1) / MB;
#pragma omp parallel for num_threads(g_orc_threads) schedule(static) if (g_orc_threads > 1)
    for (int64_t bi = 0; bi < nblk; ++bi) {
        const int64_t i0 = bi * MB;
        int64_t i1 = i0 + MB < m ? i0 + MB : m;
        float *acc = (float *)malloc(sizeof(float) * (size_t)(MB * n));
        if (!acc) continue; /* cannot happen at the sizes used; leaves C unchanged */
        memset(acc, 0, sizeof(float) * (size_t)((i1 - i0) * n));
        for (int64_t p0 = 0; p0 < k; p0 += KB) {
            int64_t p1 = p0 + KB < k ? p0 + KB : k;
            for (int64_t i = i0; i < i1; ++i) {
                float *ar = &acc[(i - i0) * n];
                const float *a = &A[i * lda];
                for (int64_t p = p0; p < p1; ++p) {
                    float av = a[p];
                    const float *b = &B[p * ldb];
                    for (int64_t j = 0; j < n; ++j) ar[j] += av * b[j];
                }
            }
        }
        for (int64_t i = i0; i < i1; ++i)
            for (int64_t j = 0; j < n; ++j) C[i * ldc + j] += acc[(i - i0) * n + j];
        free(acc);
    }
}

/*
 * sparse_subm_conv_forward_flex_precomputed,
 * crates/burn_flex_gmm/src/lib.rs:242-375: out = bias; per group gather an
 * im2col [n_q, K*Cin_g] (zeros where the neighbour is -1) and out += im2col @
 * packed.  input is [n_in, Cin] with n_in >= n_q; nbr is [n_q, K].
 * packed may be NULL (then pack_flex_weight is applied, :313-316).
 */
int orc_conv_flex_precomputed(const orc_cfg *c, const float *w, const float *bias,
                              const float *input, int64_t n_in, const int32_t *nbr,
                              int64_t n_q, const float *packed_in, float *out)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    if (n_in < n_q) return ORC_ERR_SHAPE;
    if (n_q == 0) return ORC_OK;
    int64_t K = orc_kernel_rows(c), cin = c->in_channels_per_group,
            n = c->out_channels_per_group, kin = K * cin, C_in = c->in_channels,
            C_out = c->out_channels;
    float *packed_own = NULL;
    const float *packed = packed_in;
    if (!packed) {
        packed_own = (float *)malloc(sizeof(float) * (size_t)(c->groups * kin * n));
        if (!packed_own) return ORC_ERR_ALLOC;
        orc_pack_flex_weight(c, w, packed_own);
        packed = packed_own;
    }
    for (int64_t r = 0; r < n_q; ++r) memcpy(&out[r * C_out], bias, sizeof(float) * (size_t)C_out);
    float *g_buf = (float *)malloc(sizeof(float) * (size_t)(n_q * kin));
    if (!g_buf) {
        free(packed_own);
        return ORC_ERR_ALLOC;
    }
    int rc = ORC_OK;
    for (int64_t g = 0; g < c->groups && rc == ORC_OK; ++g) {
        memset(g_buf, 0, sizeof(float) * (size_t)(n_q * kin));
        int bad = 0;
#pragma omp parallel for num_threads(g_orc_threads) schedule(static) reduction(| : bad) if (g_orc_threads > 1)
        for (int64_t r = 0; r < n_q; ++r)
            for (int64_t k = 0; k < K; ++k) {
                int32_t s = nbr[r * K + k];
                if (s == ORC_INVALID_NEIGHBOR) continue;
                if (s < 0 || s >= n_in) {
                    bad = 1;
                    continue;
                }
                memcpy(&g_buf[r * kin + k * cin], &input[(int64_t)s * C_in + g * cin],
                       sizeof(float) * (size_t)cin);
            }
        if (bad) rc = ORC_ERR_INDEX;
        if (rc == ORC_OK)
            orc_sgemm_acc(n_q, kin, n, g_buf, kin, &packed[g * kin * n], n, &out[g * n], C_out);
    }
    free(g_buf);
    free(packed_own);
    return rc;
}

/*
 * sparse_subm_conv_forward_legacy, crates/burn_flex_gmm/src/lib.rs:428-510:
 * the direct nested-loop definition, with its own coord->row HashMap (last
 * duplicate wins, :446-449) and offset walk (:455-479).
 */
int orc_conv_legacy(const orc_cfg *c, const float *w, const float *bias, const uint32_t *coords,
                    int64_t n, const float *input, float *out)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    if (n == 0) return ORC_OK;
    int64_t C_in = c->in_channels, C_out = c->out_channels, cin = c->in_channels_per_group,
            cout = c->out_channels_per_group;
    for (int64_t r = 0; r < n; ++r) memcpy(&out[r * C_out], bias, sizeof(float) * (size_t)C_out);
    orc_map m;
    if (orc_map_init(&m, n) != ORC_OK) return ORC_ERR_ALLOC;
    for (int64_t r = 0; r < n; ++r) orc_map_insert_last(&m, &coords[4 * r], r);
    int32_t cd = (int32_t)(c->kernel_d / 2), ch = (int32_t)(c->kernel_h / 2),
            cw = (int32_t)(c->kernel_w / 2);
    for (int64_t r = 0; r < n; ++r) {
        const uint32_t *q = &coords[4 * r];
        for (int64_t kd = 0; kd < c->kernel_d; ++kd)
            for (int64_t kh = 0; kh < c->kernel_h; ++kh)
                for (int64_t kw = 0; kw < c->kernel_w; ++kw) {
                    int32_t d[3] = {c->axis_sign[0] * ((int32_t)kd - cd),
                                    c->axis_sign[1] * ((int32_t)kh - ch),
                                    c->axis_sign[2] * ((int32_t)kw - cw)};
                    int32_t sp[3] = {(int32_t)q[1], (int32_t)q[2], (int32_t)q[3]};
                    sp[c->axis_order[0]] += d[0];
                    sp[c->axis_order[1]] += d[1];
                    sp[c->axis_order[2]] += d[2];
                    if (sp[0] < 0 || sp[1] < 0 || sp[2] < 0) continue;
                    uint32_t key[4] = {q[0], (uint32_t)sp[0], (uint32_t)sp[1], (uint32_t)sp[2]};
                    int64_t s = orc_map_get(&m, key);
                    if (s < 0) continue;
                    const float *in_row = &input[s * C_in];
                    for (int64_t g = 0; g < c->groups; ++g)
                        for (int64_t ol = 0; ol < cout; ++ol) {
                            int64_t o = g * cout + ol;
                            const float *wr =
                                &w[(((o * c->kernel_d + kd) * c->kernel_h + kh) * c->kernel_w + kw) *
                                   cin];
                            float acc = 0.0f;
                            for (int64_t i = 0; i < cin; ++i) acc += in_row[g * cin + i] * wr[i];
                            out[r * C_out + o] += acc;
                        }
                }
    }
    orc_map_free(&m);
    return ORC_OK;
}

/*
 * fp64 evaluation of the same definition over a precomputed map (the sum of
 * crates/burn_flex_gmm/src/wgpu/sparse_conv_kernels.rs:5-46: bias first, skip
 * invalid neighbours).  Operands are read as given (already rounded to bf16
 * or dequantised by the caller); out is [n_q, Cout] in double.
 * w_scale (nullable) multiplies output channel o after the sum (int8
 * per-output-channel weights).
 */
int orc_conv_ref_f64(const orc_cfg *c, const float *w, const float *w_scale, const float *bias,
                     const float *input, int64_t n_in, const int32_t *nbr, int64_t n_q,
                     double *out)
{
    if (orc_validate_config(c) != ORC_OK) return ORC_ERR_CONFIG;
    int64_t K = orc_kernel_rows(c), C_in = c->in_channels, C_out = c->out_channels,
            cin = c->in_channels_per_group, cout = c->out_channels_per_group;
    for (int64_t r = 0; r < n_q; ++r)
        for (int64_t o = 0; o < C_out; ++o) {
            int64_t g = o / cout;
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                int32_t s = nbr[r * K + k];
                if (s == ORC_INVALID_NEIGHBOR) continue;
                if (s < 0 || s >= n_in) return ORC_ERR_INDEX;
                const float *a = &input[(int64_t)s * C_in + g * cin];
                const float *wr = &w[(o * K + k) * cin];
                for (int64_t i = 0; i < cin; ++i) acc += (double)a[i] * (double)wr[i];
            }
            if (w_scale) acc *= (double)w_scale[o];
            out[r * C_out + o] = acc + (double)bias[o];
        }
    return ORC_OK;
}

/* bf16_round_to_f32, crates/burn_flex_gmm/src/wgpu.rs:57-67:
 * (bits + 0x7fff + ((bits>>16)&1)) & 0xffff0000, no NaN special case. */
void orc_bf16_round(const float *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        uint32_t b;
        memcpy(&b, &in[i], 4);
        uint32_t lsb = (b >> 16) & 1u;
        uint32_t r = (b + 0x7fffu + lsb) & 0xffff0000u;
        memcpy(&out[i], &r, 4);
    }
}

/* f32 -> IEEE binary16 -> f32 with round-to-nearest-even, subnormals kept,
 * overflow to +-inf: quantize_f16_inplace (sparse_decoder_wgpu_ops.rs
 * :1722-1726, half::f16::from_f32(v).to_f32()) and the F32 -> F16 -> F32
 * casts of quantize_f16_tensor_wgpu (:1082-1088). */
static uint16_t f32_to_f16_bits(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e = (x >> 23) & 0xffu, m = x & 0x7fffffu;
    if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u));
    const int32_t E = (int32_t)e - 127 + 15; /* f16 biased exponent */
    if (E >= 31) return (uint16_t)(sign | 0x7c00u);
    if (E <= 0) {                            /* f16 subnormal (or zero) */
        if (E < -10) return (uint16_t)sign;  /* below half the smallest subnormal */
        const uint32_t M = m | 0x800000u;
        const int shift = 14 - E;            /* value = M * 2^(E-14) units of 2^-24 */
        uint32_t h = M >> shift;
        const uint32_t rem = M & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h; /* may carry into the smallest normal */
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)E << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* a carry may reach the inf pattern */
    return (uint16_t)(sign | h);
}

static float f16_bits_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24, exact in f32 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f16_round(const float *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = f16_bits_to_f32(f32_to_f16_bits(in[i]));
}

/*
 * layer_norm_inplace, sparse_decoder_wgpu_ops.rs:1642-1711 (burn_trellis
 * runtime_model): two-pass f32 mean and biased variance per row,
 * (x - mean) * (1/sqrt(var + eps)) [* w] [+ b].  w, b nullable.
 */
void orc_layer_norm(float *data, int64_t rows, int64_t ch, const float *w, const float *b,
                    float eps)
{
    for (int64_t r = 0; r < rows; ++r) {
        float *x = &data[r * ch];
        float sum = 0.0f;
        for (int64_t j = 0; j < ch; ++j) sum += x[j];
        float mean = sum / (float)ch;
        float sq = 0.0f;
        for (int64_t j = 0; j < ch; ++j) {
            float d = x[j] - mean;
            sq += d * d;
        }
        float var = sq / (float)ch;
        float inv = 1.0f / sqrtf(var + eps);
        for (int64_t j = 0; j < ch; ++j) {
            float v = (x[j] - mean) * inv;
            if (w) v *= w[j];
            if (b) v += b[j];
            x[j] = v;
        }
    }
}

/* silu_inplace, sparse_decoder_wgpu_ops.rs:1713-1720: x / (1 + exp(-x)). */
void orc_silu(float *data, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) data[i] = data[i] / (1.0f + expf(-data[i]));
}

/*
 * Subdivision mask + active pairs: logits_to_mask (sparse_decoder_wgpu_ops.rs
 * :1765-1811, mask[c] = logit > thr[c]) followed by the parent-major,
 * child-ascending enumeration of argwhere on [P,8] (:885-993).  pairs is
 * [A][2] (parent, child); returns A.
 */
int64_t orc_subdivision_active(const float *logits, int64_t rows, const float thr[8],
                               int32_t *pairs)
{
    int64_t a = 0;
    for (int64_t r = 0; r < rows; ++r)
        for (int c = 0; c < 8; ++c)
            if (logits[r * 8 + c] > thr[c]) {
                if (pairs) {
                    pairs[2 * a] = (int32_t)r;
                    pairs[2 * a + 1] = c;
                }
                ++a;
            }
    return a;
}

/*
 * expand_subdivision_coords_and_linear_indices_wgpu,
 * sparse_decoder_wgpu_ops.rs:996-1054: child = [b, 2x+(c&1), 2y+(c>>1&1),
 * 2z+(c>>2&1)], linear_idx = 8*parent + c.
 */
void orc_subdivide_expand(const uint32_t *parent_coords, const int32_t *pairs, int64_t a,
                          uint32_t *child_coords, int32_t *linear_idx)
{
    for (int64_t i = 0; i < a; ++i) {
        int32_t p = pairs[2 * i], c = pairs[2 * i + 1];
        const uint32_t *pc = &parent_coords[4 * (int64_t)p];
        child_coords[4 * i + 0] = pc[0];
        child_coords[4 * i + 1] = pc[1] * 2u + (uint32_t)(c & 1);
        child_coords[4 * i + 2] = pc[2] * 2u + (uint32_t)((c >> 1) & 1);
        child_coords[4 * i + 3] = pc[3] * 2u + (uint32_t)((c >> 2) & 1);
        linear_idx[i] = p * 8 + c;
    }
}

/*
 * channel2spatial, sparse_decoder_wgpu_ops.rs:1999-2054: for each parent in
 * order and each selected child c ascending, emit the child coord and the
 * feature block [c*Cout, (c+1)*Cout) of the parent row, Cout = Cin/8.
 * mask is [rows][8] u8.  Returns the child count.
 */
int64_t orc_channel2spatial(const uint32_t *coords, const float *feats, int64_t rows,
                            int64_t in_channels, const uint8_t *mask, uint32_t *out_coords,
                            float *out_feats)
{
    int64_t oc = in_channels / 8, a = 0;
    for (int64_t r = 0; r < rows; ++r)
        for (int c = 0; c < 8; ++c) {
            if (!mask[r * 8 + c]) continue;
            const uint32_t *pc = &coords[4 * r];
            out_coords[4 * a + 0] = pc[0];
            out_coords[4 * a + 1] = pc[1] * 2u + (uint32_t)(c & 1);
            out_coords[4 * a + 2] = pc[2] * 2u + (uint32_t)((c >> 1) & 1);
            out_coords[4 * a + 3] = pc[3] * 2u + (uint32_t)((c >> 2) & 1);
            memcpy(&out_feats[a * oc], &feats[r * in_channels + c * oc], sizeof(float) * (size_t)oc);
            ++a;
        }
    return a;
}

/* repeat_interleave_channels, sparse_decoder_wgpu_ops.rs:2056-2076. */
void orc_repeat_interleave(const float *feats, int64_t rows, int64_t ch, int64_t rep, float *out)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < ch; ++j)
            for (int64_t t = 0; t < rep; ++t) out[(r * ch + j) * rep + t] = feats[r * ch + j];
}

/*
 * The C2S upsample block on the host, sparse_decoder_runtime_impl.rs
 * :1236-1343 (fp16 fences off): h = SiLU(LN(parent; norm1 w,b)); conv1 on
 * parent coords (Cin -> 8*Cout); channel2spatial of conv1 output and of the
 * parent features (skip); h_up = SiLU(LN(children; no affine)); conv2 on the
 * child coords; out = conv2 + repeat_interleave(skip, Cout/(Cin/8)).
 * Convolutions use the flex path over maps built by orc_build_neighbor_rows.
 * Children are produced in the order of orc_channel2spatial.  Returns the
 * child count or a negative error.
 */
int64_t orc_c2s_block(const uint32_t *parent_coords, const float *parent_feats, int64_t p_rows,
                      int64_t in_ch, int64_t out_ch, const uint8_t *mask, const float *norm1_w,
                      const float *norm1_b, const orc_cfg *conv1, const float *w1, const float *b1,
                      const orc_cfg *conv2, const float *w2, const float *b2, float eps,
                      uint32_t *child_coords, float *out)
{
    int64_t K1 = orc_kernel_rows(conv1), K2 = orc_kernel_rows(conv2);
    if (K1 < 0 || K2 < 0) return -ORC_ERR_CONFIG;
    if (conv1->in_channels != in_ch || conv1->out_channels != 8 * out_ch ||
        conv2->in_channels != out_ch || conv2->out_channels != out_ch || in_ch % 8 != 0 ||
        out_ch % (in_ch / 8) != 0)
        return -ORC_ERR_SHAPE;
    float *h = (float *)malloc(sizeof(float) * (size_t)(p_rows * in_ch));
    float *h1 = (float *)malloc(sizeof(float) * (size_t)(p_rows * 8 * out_ch));
    int32_t *nb1 = (int32_t *)malloc(sizeof(int32_t) * (size_t)(p_rows * K1 + 1));
    memcpy(h, parent_feats, sizeof(float) * (size_t)(p_rows * in_ch));
    orc_layer_norm(h, p_rows, in_ch, norm1_w, norm1_b, eps);
    orc_silu(h, p_rows * in_ch);
    orc_build_neighbor_rows(conv1, parent_coords, p_rows, p_rows, 0, nb1);
    orc_conv_flex_precomputed(conv1, w1, b1, h, p_rows, nb1, p_rows, NULL, h1);
    int64_t a = 0;
    for (int64_t r = 0; r < p_rows; ++r)
        for (int c = 0; c < 8; ++c) a += mask[r * 8 + c] ? 1 : 0;
    float *hup = (float *)malloc(sizeof(float) * (size_t)(a * out_ch + 1));
    float *xup = (float *)malloc(sizeof(float) * (size_t)(a * (in_ch / 8) + 1));
    uint32_t *cc2 = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(a * 4 + 1));
    orc_channel2spatial(parent_coords, h1, p_rows, 8 * out_ch, mask, child_coords, hup);
    orc_channel2spatial(parent_coords, parent_feats, p_rows, in_ch, mask, cc2, xup);
    orc_layer_norm(hup, a, out_ch, NULL, NULL, eps);
    orc_silu(hup, a * out_ch);
    int32_t *nb2 = (int32_t *)malloc(sizeof(int32_t) * (size_t)(a * K2 + 1));
    orc_build_neighbor_rows(conv2, child_coords, a, a, 0, nb2);
    orc_conv_flex_precomputed(conv2, w2, b2, hup, a, nb2, a, NULL, out);
    int64_t sc = in_ch / 8, rep = out_ch / sc;
    for (int64_t i = 0; i < a; ++i)
        for (int64_t j = 0; j < out_ch; ++j) out[i * out_ch + j] += xup[i * sc + j / rep];
    free(h);
    free(h1);
    free(nb1);
    free(hup);
    free(xup);
    free(cc2);
    free(nb2);
    return a;
}

/*
 * The 64-bit LCG the reference's tests use to make inputs,
 * crates/burn_flex_gmm/src/lib.rs:764-778 (copies in wgpu/tests.rs:47-61 and
 * sparse_decoder_tests.rs:170-186): state = seed|1; state = state*
 * 6364136223846793005 + 1; bits = (state>>40)|1; (bits/u32::MAX)*2-1 in f32.
 * Fills n values; returns the final state so that a sequence can continue.
 */
uint64_t orc_lcg_fill(uint64_t state, int64_t n, float *out)
{
    for (int64_t i = 0; i < n; ++i) {
        state = state * 6364136223846793005ull + 1ull;
        uint32_t bits = (uint32_t)(state >> 40) | 1u;
        volatile float q = (float)bits / (float)UINT32_MAX;
        out[i] = q * 2.0f - 1.0f;
    }
    return state;
}
