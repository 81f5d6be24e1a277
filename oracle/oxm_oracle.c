/*
 * oxm_oracle.c -- CPU restatement of oxmera's reference matmul.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP GEMM
 * backend: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product library (oxmera_amd/liboxm.so) never links
 * or calls it.
 *
 * What it restates (the reference's bodies are todo!(), so the contract is
 * the A4 spec and the ops/core documentation):
 *   - CpuBackend::matmul            crates/oxmera-cpu/src/lib.rs:71-76
 *       "three nested loops you can prove correct"
 *                                   exercises/a4-reference-matmul/README.md:7-19
 *       reads through views         exercises/a4-reference-matmul/tests/spec.rs:85-94
 *   - MatmulOps::matmul contract    crates/oxmera-ops/src/lib.rs:9-19,52-59
 *       [m,k]x[k,n]->[m,n], fresh contiguous output.
 *   - Layout::offset_of             crates/oxmera-core/src/layout.rs:24-49
 *       offset + sum(idx_d * stride_d), element strides, signed.
 *   - broadcast_shapes              crates/oxmera-core/src/shape.rs:45-58
 *       NumPy rules, applied to the batch dims (everything but the last two).
 * Extensions this build defines (the reference has no BF16/F16, no batched
 * matmul and no fused epilogue yet, crates/oxmera-core/src/dtype.rs:9-22):
 *   - bf16 / f16 operands are widened exactly to f32;
 *   - accumulation is f32, ascending k;
 *   - epilogue: pre = acc + bias[n]; act NONE / GELU(erf) (aux = pre) /
 *     DGELU (acc * GELU'(aux[m,n])) / GELU_GRAD (GELU(pre), aux = GELU'(pre))
 *     / MUL_AUX (acc * aux[m,n]); outputs are rounded once to their dtype
 *     (round-to-nearest-even for bf16/f16).
 *
 * Pinning: tests/test_oracle.py checks every function here against the A4
 * hand-computed products, identity/zero laws, transposed-view read, transpose
 * law and column independence, against numpy float64 golden fixtures under
 * tests/golden/, against closed forms (ones*ones = K, rank-1 outer products,
 * diagonal scaling) and against scipy's erf for the GELU epilogue.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_F32 = 0, OR_F64 = 1, OR_I32 = 2, OR_I64 = 3, OR_U8 = 4, OR_BOOL = 5, OR_BF16 = 6, OR_F16 = 7 };
enum { OR_ACT_NONE = 0, OR_ACT_GELU = 1, OR_ACT_DGELU = 2, OR_ACT_GELU_GRAD = 3, OR_ACT_MUL_AUX = 4 };
enum { OR_OK = 0, OR_E_SHAPE = 1, OR_E_BROADCAST = 2, OR_E_DTYPE = 3, OR_E_UNSUPPORTED = 4, OR_E_RANK = 7 };

#define OR_MAXDIM 8

/* Same memory layout as the product's oxm_view; declared separately so the
 * oracle shares no code with the library it checks. */
typedef struct {
    void *data;
    int32_t dtype;
    int32_t ndim;
    const int64_t *shape;
    const int64_t *strides; /* elements, signed (layout.rs:6-10) */
    int64_t offset;         /* elements (layout.rs:31-33) */
    int32_t device;
} or_view;

/* ---- scalar conversions ------------------------------------------------ */

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);                                           /* RNE */
    return (uint16_t)(u >> 16);
}

/* IEEE binary16 <-> binary32, written from the format definition. */
static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    int32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (exp == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float f = (float)man * 5.9604644775390625e-08f;
            memcpy(&u, &f, 4);
            u |= sign;
        }
    } else {
        u = sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;          /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u;         /* rounds to inf (>= 65520) */
    if (a < 0x38800000u) {                               /* below 2^-14: subnormal */
        float af;
        memcpy(&af, &a, 4);
        /* value / 2^-24 rounded to nearest even (default FP rounding mode) */
        float q = nearbyintf(af * 16777216.0f);
        return sign | (uint16_t)q;
    }
    uint32_t r = a + 0xfffu + ((a >> 13) & 1u); /* RNE on the 13 dropped bits */
    return sign | (uint16_t)((r - 0x38000000u) >> 13);
}

static float load_f(const void *base, int dtype, int64_t idx) {
    switch (dtype) {
    case OR_F32: return ((const float *)base)[idx];
    case OR_F64: return (float)((const double *)base)[idx];
    case OR_BF16: return bf16_to_f32(((const uint16_t *)base)[idx]);
    case OR_F16: return f16_to_f32(((const uint16_t *)base)[idx]);
    default: return 0.0f;
    }
}

static void store_f(void *base, int dtype, int64_t idx, float v) {
    switch (dtype) {
    case OR_F32: ((float *)base)[idx] = v; break;
    case OR_F64: ((double *)base)[idx] = (double)v; break;
    case OR_BF16: ((uint16_t *)base)[idx] = f32_to_bf16(v); break;
    case OR_F16: ((uint16_t *)base)[idx] = f32_to_f16(v); break;
    default: break;
    }
}

/* GELU with the exact (erf) form: x * Phi(x). */
static float gelu_f(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }

/* d/dx [x * Phi(x)] = Phi(x) + x * phi(x). */
static float dgelu_f(float x) {
    float cdf = 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
    float pdf = expf(-0.5f * x * x) * 0.39894228040143267794f; /* 1/sqrt(2*pi) */
    return cdf + x * pdf;
}

/* Exported for the tests that pin the epilogue against scipy's erf. */
float oxm_oracle_gelu(float x) { return gelu_f(x); }
float oxm_oracle_dgelu(float x) { return dgelu_f(x); }
uint16_t oxm_oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }
float oxm_oracle_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
uint16_t oxm_oracle_f32_to_f16(float f) { return f32_to_f16(f); }
float oxm_oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* ---- shapes ------------------------------------------------------------- */

/* broadcast_shapes (shape.rs:45-58): align trailing dims; each pair equal or
 * one of them 1.  Returns OR_E_BROADCAST on refusal. */
int oxm_oracle_broadcast(int na, const int64_t *a, int nb, const int64_t *b, int *nout, int64_t *out) {
    int n = na > nb ? na : nb;
    for (int i = 0; i < n; ++i) {
        int ia = na - n + i, ib = nb - n + i;
        int64_t da = ia >= 0 ? a[ia] : 1, db = ib >= 0 ? b[ib] : 1;
        if (da == db || db == 1) out[i] = da;
        else if (da == 1) out[i] = db;
        else return OR_E_BROADCAST;
    }
    *nout = n;
    return OR_OK;
}

/* ---- the matmul ------------------------------------------------------- */

typedef struct {
    const or_view *a, *b;
    int nbatch;              /* number of output batch dims */
    int64_t bshape[OR_MAXDIM];
    int64_t bsa[OR_MAXDIM];  /* a's stride for each output batch dim (0 = broadcast) */
    int64_t bsb[OR_MAXDIM];
    int64_t M, N, K;
    int64_t sam, sak, sbk, sbn;
    int out_dtype;
    const void *bias;
    int bias_dtype;
    int act;
    void *aux;               /* DGELU: Z input; MUL_AUX: the factor (out_dtype) */
    const int64_t *rows;     /* flattened (batch*M + m) rows to compute, NULL = all */
    int64_t nrows;
    void *out;               /* [nrows, N] (rows given) or the full [batch..., M, N] */
    void *aux_rows;          /* same indexing as out */
} job_t;

typedef struct {
    const job_t *job;
    int64_t r0, r1;
} slice_t;

static void compute_row(const job_t *j, int64_t flat, int64_t out_row) {
    int64_t bidx = flat / j->M, m = flat % j->M;
    int64_t offa = j->a->offset, offb = j->b->offset;
    /* unravel the batch index, last batch dim fastest */
    int64_t rem = bidx;
    for (int d = j->nbatch - 1; d >= 0; --d) {
        int64_t i = rem % j->bshape[d];
        rem /= j->bshape[d];
        offa += i * j->bsa[d];
        offb += i * j->bsb[d];
    }
    for (int64_t n = 0; n < j->N; ++n) {
        float acc = 0.0f;
        for (int64_t k = 0; k < j->K; ++k) { /* ascending k, f32 accumulate */
            float x = load_f(j->a->data, j->a->dtype, offa + m * j->sam + k * j->sak);
            float y = load_f(j->b->data, j->b->dtype, offb + k * j->sbk + n * j->sbn);
            acc += x * y;
        }
        int64_t o = out_row * j->N + n;
        float v = acc;
        if (j->act == OR_ACT_DGELU) {
            float z = load_f(j->aux, j->out_dtype, flat * j->N + n);
            v = acc * dgelu_f(z);
        } else if (j->act == OR_ACT_MUL_AUX) {
            v = acc * load_f(j->aux, j->out_dtype, flat * j->N + n);
        } else {
            if (j->bias) v = acc + load_f(j->bias, j->bias_dtype, n);
            if (j->act == OR_ACT_GELU) {
                if (j->aux_rows) store_f(j->aux_rows, j->out_dtype, o, v);
                v = gelu_f(v);
            } else if (j->act == OR_ACT_GELU_GRAD) {
                if (j->aux_rows) store_f(j->aux_rows, j->out_dtype, o, dgelu_f(v));
                v = gelu_f(v);
            }
        }
        store_f(j->out, j->out_dtype, o, v);
    }
}

static void *run_slice(void *arg) {
    const slice_t *s = (const slice_t *)arg;
    for (int64_t r = s->r0; r < s->r1; ++r) {
        int64_t flat = s->job->rows ? s->job->rows[r] : r;
        compute_row(s->job, flat, r);
    }
    return NULL;
}

/*
 * oxm_oracle_gemm: C = epilogue(A . B) over broadcast batch dims.
 *   rows == NULL : compute every output row into `out` (contiguous
 *                  [batch..., M, N]); aux_out likewise.
 *   rows != NULL : compute only the listed flattened rows (b*M + m) into
 *                  out[nrows, N] (the sampled check for 8192^3 shapes).
 * Validation mirrors MatmulOps::matmul: rank >= 2 (rank-1 refused,
 * a4 spec.rs:78-83), inner dims equal (ShapeMismatch, spec.rs:68-76),
 * same dtype (DTypeMismatch, ops/src/lib.rs:13-15), batch dims broadcast.
 */
int oxm_oracle_gemm(const or_view *a, const or_view *b, int out_dtype, const void *bias, int bias_dtype,
                    int act, void *aux, const int64_t *rows, int64_t nrows, void *out, void *aux_out,
                    int nthreads) {
    if (a->ndim < 2 || b->ndim < 2) return OR_E_RANK;
    if (a->dtype != b->dtype) return OR_E_DTYPE;
    if (!(a->dtype == OR_F32 || a->dtype == OR_BF16 || a->dtype == OR_F16 || a->dtype == OR_F64))
        return OR_E_UNSUPPORTED;
    if (a->ndim > OR_MAXDIM || b->ndim > OR_MAXDIM) return OR_E_RANK;
    job_t j;
    memset(&j, 0, sizeof j);
    j.a = a;
    j.b = b;
    j.M = a->shape[a->ndim - 2];
    j.K = a->shape[a->ndim - 1];
    j.N = b->shape[b->ndim - 1];
    if (b->shape[b->ndim - 2] != j.K) return OR_E_SHAPE;
    j.sam = a->strides[a->ndim - 2];
    j.sak = a->strides[a->ndim - 1];
    j.sbk = b->strides[b->ndim - 2];
    j.sbn = b->strides[b->ndim - 1];
    int nb;
    if (oxm_oracle_broadcast(a->ndim - 2, a->shape, b->ndim - 2, b->shape, &nb, j.bshape) != OR_OK)
        return OR_E_BROADCAST;
    j.nbatch = nb;
    for (int d = 0; d < nb; ++d) {
        int da = a->ndim - 2 - nb + d, db = b->ndim - 2 - nb + d;
        j.bsa[d] = (da >= 0 && a->shape[da] != 1) ? a->strides[da] : 0;
        j.bsb[d] = (db >= 0 && b->shape[db] != 1) ? b->strides[db] : 0;
    }
    int64_t batch = 1;
    for (int d = 0; d < nb; ++d) batch *= j.bshape[d];
    j.out_dtype = out_dtype;
    j.bias = bias;
    j.bias_dtype = bias_dtype;
    j.act = act;
    j.aux = aux;
    j.rows = rows;
    j.nrows = rows ? nrows : batch * j.M;
    j.out = out;
    j.aux_rows = aux_out;
    if (j.nrows == 0 || j.N == 0) return OR_OK;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (nthreads > j.nrows) nthreads = (int)j.nrows;
    pthread_t th[256];
    slice_t sl[256];
    for (int t = 0; t < nthreads; ++t) {
        sl[t].job = &j;
        sl[t].r0 = j.nrows * t / nthreads;
        sl[t].r1 = j.nrows * (t + 1) / nthreads;
    }
    for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, run_slice, &sl[t]);
    run_slice(&sl[0]);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
    return OR_OK;
}

/*
 * Column sum over the rows of a contiguous [R, C] matrix (bias gradient,
 * ReduceOps::sum over axis 0, ops/src/lib.rs:61-69), f32 accumulate in
 * ascending row order.
 */
void oxm_oracle_colsum(const void *x, int dtype, int64_t R, int64_t C, float *out) {
    for (int64_t c = 0; c < C; ++c) {
        float s = 0.0f;
        for (int64_t r = 0; r < R; ++r) s += load_f(x, dtype, r * C + c);
        out[c] = s;
    }
}
