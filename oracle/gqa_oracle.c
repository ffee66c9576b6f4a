/*
 * gqa_oracle.c -- CPU restatement of the reference golden model for the GQA
 * attention step.  TEST INFRASTRUCTURE ONLY: tests/, the smoke check and the
 * benchmark's CPU-baseline leg call it as the checker; the product path never
 * links or calls it.
 *
 * Arithmetic follows the reference's pure-Python golden exactly, in IEEE double
 * with no contraction (built with -ffp-contract=off), glibc libm for
 * pow/cos/sin/exp (what CPython's math module and float ** call):
 *
 *   rope_half_split        pyfiles/gen_gqa_wrapper_vectors.py:25-35
 *   golden attention loop  pyfiles/gen_gqa_wrapper_vectors.py:121-139
 *   f32_to_bf16            pyfiles/gqa_reference.py:15-19
 *
 * Python's built-in sum() differs by interpreter version: CPython <= 3.11 adds
 * floats left to right; CPython >= 3.12 uses Neumaier-compensated summation
 * (Neumaier 1974, "Rundungsfehleranalyse einiger Verfahren zur Summation
 * endlicher Summen").  ORACLE_SUM_SEQUENTIAL / ORACLE_SUM_NEUMAIER select which
 * interpreter's golden is restated; the two differ only in the last bits of a
 * double, which BF16 output rounding absorbs except at exact ties.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define ORACLE_SUM_SEQUENTIAL 0
#define ORACLE_SUM_NEUMAIER 1

typedef struct {
    double sum;
    double comp;
    int mode;
    int started;
} py_sum_t;

static inline void pysum_init(py_sum_t* s, int mode) {
    s->sum = 0.0;
    s->comp = 0.0;
    s->mode = mode;
    s->started = 0;
}

/* sum(iterable) with the default int start 0: the first float replaces the int
 * (0 + x == x for every finite x of interest), then floats accumulate. */
static inline void pysum_add(py_sum_t* s, double x) {
    if (!s->started) {
        s->sum = 0.0 + x;
        s->started = 1;
        return;
    }
    if (s->mode == ORACLE_SUM_NEUMAIER) {
        double t = s->sum + x;
        if (fabs(s->sum) >= fabs(x))
            s->comp += (s->sum - t) + x;
        else
            s->comp += (x - t) + s->sum;
        s->sum = t;
    } else {
        s->sum += x;
    }
}

static inline double pysum_result(const py_sum_t* s) {
    if (s->mode == ORACLE_SUM_NEUMAIER && s->comp != 0.0 && isfinite(s->comp))
        return s->sum + s->comp;
    return s->sum;
}

/* pyfiles/gqa_reference.py:15-19: double -> f32 (RNE, the struct.pack('>f') cast)
 * -> BF16 by (bits + 0x7FFF + lsb) >> 16.  Returns -1 where struct.pack would
 * raise OverflowError (finite double beyond the f32 range). */
int32_t oracle_f32_to_bf16(double value) {
    float f = (float)value;
    if (isinf(f) && !isinf(value))
        return -1;
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t lsb = (bits >> 16) & 1u;
    return (int32_t)(((uint64_t)bits + 0x7FFFu + lsb) >> 16 & 0xFFFFu);
}

/* pyfiles/gqa_reference.py:22-23 */
double oracle_bf16_to_f64(uint16_t bits) {
    uint32_t w = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &w, 4);
    return (double)f;
}

/* pyfiles/gen_gqa_wrapper_vectors.py:25-35.  angle = position * theta**(-2i/n),
 * out[i] = x*c - y*s, out[i+n/2] = x*s + y*c; nothing re-rounded. */
void oracle_rope_half_split(const double* row, int n, int64_t position, double theta,
                            double* out) {
    int half = n / 2;
    if (out != row)
        memcpy(out, row, sizeof(double) * (size_t)n);
    for (int i = 0; i < half; ++i) {
        double e = (-2.0 * (double)i) / (double)n;
        double angle = (double)position * pow(theta, e);
        double c = cos(angle), s = sin(angle);
        double x = row[i], y = row[i + half];
        out[i] = x * c - y * s;
        out[i + half] = x * s + y * c;
    }
}

/* Widen BF16 rows to double and optionally rotate each at position pos0 + r.
 * rows: [n_rows] rows of n elements, row stride `stride` elements. */
void oracle_prepare_rows(const uint16_t* rows, int64_t n_rows, int64_t stride, int n,
                         int rotate, int64_t pos0, double theta, double* out) {
    double* tmp = (double*)malloc(sizeof(double) * (size_t)n);
    for (int64_t r = 0; r < n_rows; ++r) {
        for (int d = 0; d < n; ++d)
            tmp[d] = oracle_bf16_to_f64(rows[r * stride + d]);
        if (rotate)
            oracle_rope_half_split(tmp, n, pos0 + r, theta, out + r * n);
        else
            memcpy(out + r * n, tmp, sizeof(double) * (size_t)n);
    }
    free(tmp);
}

/* The golden loop of pyfiles/gen_gqa_wrapper_vectors.py:130-139 for one query
 * token, on already-prepared double rows:
 *   q_ref   [q_heads][d]
 *   k_ref   [kv_heads][key_stride][d]   (rows 0..n_keys-1 used)
 *   v_ref   [kv_heads][key_stride][d]
 * n_keys = query_position + 1 (keys p <= query_position; the generator enforces
 * query_position < seq_len, so the padding mask p < seq_len is implied).
 * out_bf16 [q_heads][d] (may be NULL), out_f64 [q_heads][d] (may be NULL).
 * Returns 0, or -1 if an output overflows f32 (the OverflowError case). */
int oracle_attend(int q_heads, int kv_heads, int d, const double* q_ref, const double* k_ref,
                  const double* v_ref, int64_t key_stride, int64_t n_keys, double scale,
                  int sum_mode, uint16_t* out_bf16, double* out_f64) {
    int group = q_heads / kv_heads;
    double* scores = (double*)malloc(sizeof(double) * (size_t)n_keys);
    double* weights = (double*)malloc(sizeof(double) * (size_t)n_keys);
    py_sum_t* accs = (py_sum_t*)malloc(sizeof(py_sum_t) * (size_t)d);
    double* plain = (double*)malloc(sizeof(double) * (size_t)d);
    int status = 0;
    for (int qh = 0; qh < q_heads; ++qh) {
        int kh = qh / group;
        const double* q = q_ref + (int64_t)qh * d;
        const double* kb = k_ref + (int64_t)kh * key_stride * d;
        const double* vb = v_ref + (int64_t)kh * key_stride * d;
        if (sum_mode == ORACLE_SUM_SEQUENTIAL) {
            /* Left-to-right sums; four keys in flight for ILP, each its own chain. */
            int64_t p = 0;
            for (; p + 4 <= n_keys; p += 4) {
                const double* k0 = kb + p * d;
                double a0 = q[0] * k0[0], a1 = q[0] * k0[d], a2 = q[0] * k0[2 * d],
                       a3 = q[0] * k0[3 * d];
                for (int j = 1; j < d; ++j) {
                    a0 += q[j] * k0[j];
                    a1 += q[j] * k0[d + j];
                    a2 += q[j] * k0[2 * d + j];
                    a3 += q[j] * k0[3 * d + j];
                }
                scores[p] = a0 * scale;
                scores[p + 1] = a1 * scale;
                scores[p + 2] = a2 * scale;
                scores[p + 3] = a3 * scale;
            }
            for (; p < n_keys; ++p) {
                const double* k = kb + p * d;
                double a = q[0] * k[0];
                for (int j = 1; j < d; ++j)
                    a += q[j] * k[j];
                scores[p] = a * scale;
            }
        } else {
            for (int64_t p = 0; p < n_keys; ++p) {
                py_sum_t s;
                pysum_init(&s, sum_mode);
                const double* k = kb + p * d;
                for (int j = 0; j < d; ++j)
                    pysum_add(&s, q[j] * k[j]);
                scores[p] = pysum_result(&s) * scale;
            }
        }
        double mx = scores[0];
        for (int64_t p = 1; p < n_keys; ++p)
            if (scores[p] > mx)
                mx = scores[p];
        py_sum_t norm;
        pysum_init(&norm, sum_mode);
        for (int64_t p = 0; p < n_keys; ++p) {
            weights[p] = exp(scores[p] - mx);
            pysum_add(&norm, weights[p]);
        }
        double normalizer = pysum_result(&norm);
        /* sum(weights[p] * v[p][j] for p ...) for every j: each j keeps its own running
         * sum, visited in increasing p, so the per-element addition order is the
         * reference's; only the loop nest is swapped for row-order memory access. */
        if (sum_mode == ORACLE_SUM_SEQUENTIAL) {
            for (int j = 0; j < d; ++j)
                plain[j] = weights[0] * vb[j];
            for (int64_t p = 1; p < n_keys; ++p) {
                const double w = weights[p];
                const double* vr = vb + p * d;
                for (int j = 0; j < d; ++j)
                    plain[j] += w * vr[j];
            }
        } else {
            for (int j = 0; j < d; ++j)
                pysum_init(&accs[j], sum_mode);
            for (int64_t p = 0; p < n_keys; ++p) {
                const double w = weights[p];
                const double* vr = vb + p * d;
                for (int j = 0; j < d; ++j)
                    pysum_add(&accs[j], w * vr[j]);
            }
            for (int j = 0; j < d; ++j)
                plain[j] = pysum_result(&accs[j]);
        }
        for (int j = 0; j < d; ++j) {
            double val = plain[j] / normalizer;
            if (out_f64)
                out_f64[(int64_t)qh * d + j] = val;
            if (out_bf16) {
                int32_t b = oracle_f32_to_bf16(val);
                if (b < 0) {
                    status = -1;
                    b = 0x7FC0;
                }
                out_bf16[(int64_t)qh * d + j] = (uint16_t)b;
            }
        }
    }
    free(scores);
    free(weights);
    free(accs);
    free(plain);
    return status;
}
