/*
 * Jade FP64 CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Built with -ffp-contract=off so FP32/FP64 expressions round exactly as the
 * reference's Rust source writes them (Rust never contracts a*b+c into fma).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int clamp_threads(int threads) { return threads < 1 ? 1 : threads; }

uint32_t or_xorshift32(uint32_t state) {
    state ^= state << 13;
    state ^= state >> 17;
    state ^= state << 5;
    return state;
}

void or_values(float *out, size_t len, uint32_t seed, float scale) {
    uint32_t state = seed;
    for (size_t i = 0; i < len; ++i) {
        state = or_xorshift32(state);
        const float unit = (float)(state >> 8) / 16777216.0f * 2.0f - 1.0f;
        out[i] = unit * scale;
    }
}

void or_fill(float *out, size_t len, uint32_t seed) {
    uint32_t state = seed;
    for (size_t i = 0; i < len; ++i) {
        state = or_xorshift32(state);
        out[i] = ((float)(state >> 8) / 16777216.0f) * 2.0f - 1.0f;
    }
}

void or_normal(float *out, size_t len, uint32_t seed, float mean, float sigma) {
    const double two_pi = 6.283185307179586476925286766559;
    uint32_t state = seed;
    for (size_t i = 0; i < len; ++i) {
        state = or_xorshift32(state);
        const double u1 = ((double)(state >> 8) + 1.0) / 16777216.0;
        state = or_xorshift32(state);
        const double u2 = (double)(state >> 8) / 16777216.0;
        const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)((double)mean + (double)sigma * z);
    }
}

void or_gemm_reference(uint32_t m, uint32_t n, uint32_t k, const float *a,
                       const float *b, double *out, uint32_t row0,
                       uint32_t row1, int threads) {
    (void)m;
    const long first = (long)row0, last = (long)row1;
#pragma omp parallel for num_threads(clamp_threads(threads)) schedule(dynamic, 1)
    for (long row = first; row < last; ++row) {
        double *dst = out + (size_t)(row - first) * n;
        memset(dst, 0, sizeof(double) * n);
        for (size_t p = 0; p < k; ++p) {
            const double av = (double)a[(size_t)row * k + p];
            const float *brow = b + p * (size_t)n;
            for (size_t col = 0; col < n; ++col) dst[col] += av * (double)brow[col];
        }
    }
}

void or_dot(size_t m, size_t n, size_t k, const double *a, const double *b,
            double *out, int threads) {
    const long total = (long)(m * n);
#pragma omp parallel for num_threads(clamp_threads(threads)) schedule(static)
    for (long i = 0; i < total; ++i) {
        const size_t row = (size_t)i / n, col = (size_t)i % n;
        double sum = 0.0;
        for (size_t p = 0; p < k; ++p) sum += a[row * k + p] * b[p * n + col];
        out[i] = sum;
    }
}

int or_attention_reference(uint32_t heads, uint32_t seq, uint32_t dim,
                            int causal, const float *q, const float *k,
                            const float *v, double *out, uint32_t row0,
                            uint32_t row1, int threads) {
    const size_t rows_per_head = (size_t)(row1 - row0);
    const long total = (long)((size_t)heads * rows_per_head);
    const double root = sqrt((double)dim);
    int failed = 0;
#pragma omp parallel num_threads(clamp_threads(threads))
    {
        double *scores = (double *)malloc(sizeof(double) * (seq ? seq : 1));
        if (!scores) {
#pragma omp atomic write
            failed = 1;
        }
#pragma omp for schedule(dynamic, 1)
        for (long item = 0; item < total; ++item) {
            if (!scores) continue;
            const size_t h = (size_t)item / rows_per_head;
            const size_t row = row0 + (size_t)item % rows_per_head;
            const size_t count = causal ? row + 1 : seq;
            const float *qrow = q + (h * seq + row) * dim;
            for (size_t col = 0; col < count; ++col) {
                const float *krow = k + (h * seq + col) * dim;
                double dot = 0.0;
                for (size_t d = 0; d < dim; ++d) dot += (double)qrow[d] * (double)krow[d];
                scores[col] = dot / root;
            }
            double max = -INFINITY;
            for (size_t col = 0; col < count; ++col) max = fmax(max, scores[col]);
            double denom = 0.0;
            for (size_t col = 0; col < count; ++col) {
                scores[col] = exp(scores[col] - max);
                denom += scores[col];
            }
            double *dst = out + (h * rows_per_head + (row - row0)) * dim;
            for (size_t d = 0; d < dim; ++d) {
                double acc = 0.0;
                for (size_t col = 0; col < count; ++col)
                    acc += scores[col] / denom * (double)v[(h * seq + col) * dim + d];
                dst[d] = acc;
            }
        }
        free(scores);
    }
    return failed;
}

double or_sigmoid(double x) {
    if (x >= 0.0) return 1.0 / (1.0 + exp(-x));
    const double e = exp(x);
    return e / (1.0 + e);
}

void or_normalize(size_t rows, size_t cols, const double *x,
                  const double *weight, double eps, double *out, int threads) {
#pragma omp parallel for num_threads(clamp_threads(threads)) schedule(static)
    for (long row = 0; row < (long)rows; ++row) {
        const size_t offset = (size_t)row * cols;
        double square = 0.0;
        for (size_t c = 0; c < cols; ++c) square += x[offset + c] * x[offset + c];
        const double inv = 1.0 / sqrt(square / (double)cols + eps);
        for (size_t c = 0; c < cols; ++c) out[offset + c] = x[offset + c] * inv * weight[c];
    }
}

void or_softmax(size_t rows, size_t cols, const float *x, double *out,
                int threads) {
#pragma omp parallel for num_threads(clamp_threads(threads)) schedule(static)
    for (long row = 0; row < (long)rows; ++row) {
        const float *slice = x + (size_t)row * cols;
        float maxf = -INFINITY;
        for (size_t c = 0; c < cols; ++c) maxf = fmaxf(maxf, slice[c]);
        const double max = (double)maxf;
        double sum = 0.0;
        for (size_t c = 0; c < cols; ++c) sum += exp((double)slice[c] - max);
        for (size_t c = 0; c < cols; ++c)
            out[(size_t)row * cols + c] = exp((double)slice[c] - max) / sum;
    }
}

void or_swiglu(size_t len, const float *gate, const float *up, double *out) {
    for (size_t i = 0; i < len; ++i) {
        const double g = (double)gate[i];
        out[i] = g * or_sigmoid(g) * (double)up[i];
    }
}

int or_mlp(size_t batch, size_t width, size_t hidden, const float *x,
           const float *norm, const float *wg, const float *wu,
           const float *wd, double eps, double *out, int threads) {
    const size_t xw = batch * width, wh = width * hidden, bh = batch * hidden;
    double *xd = (double *)malloc(sizeof(double) * xw);
    double *nd = (double *)calloc(width ? width : 1, sizeof(double));
    double *wgd = (double *)malloc(sizeof(double) * wh);
    double *wud = (double *)malloc(sizeof(double) * wh);
    double *wdd = (double *)malloc(sizeof(double) * wh);
    double *normalized = (double *)malloc(sizeof(double) * xw);
    double *gate = (double *)malloc(sizeof(double) * bh);
    double *upv = (double *)malloc(sizeof(double) * bh);
    double *proj = (double *)malloc(sizeof(double) * xw);
    if (!xd || !nd || !wgd || !wud || !wdd || !normalized || !gate || !upv || !proj) {
        free(xd); free(nd); free(wgd); free(wud); free(wdd);
        free(normalized); free(gate); free(upv); free(proj);
        return 1;
    }
    for (size_t i = 0; i < xw; ++i) xd[i] = (double)x[i];
    for (size_t i = 0; i < width; ++i) nd[i] = (double)norm[i];
    for (size_t i = 0; i < wh; ++i) {
        wgd[i] = (double)wg[i];
        wud[i] = (double)wu[i];
        wdd[i] = (double)wd[i];
    }
    or_normalize(batch, width, xd, nd, eps, normalized, threads);
    or_dot(batch, hidden, width, normalized, wgd, gate, threads);
    or_dot(batch, hidden, width, normalized, wud, upv, threads);
    for (size_t i = 0; i < bh; ++i) gate[i] = gate[i] * or_sigmoid(gate[i]) * upv[i];
    or_dot(batch, width, hidden, gate, wdd, proj, threads);
    for (size_t i = 0; i < xw; ++i) out[i] = proj[i] + (double)x[i];
    free(xd); free(nd); free(wgd); free(wud); free(wdd);
    free(normalized); free(gate); free(upv); free(proj);
    return 0;
}

void or_compare(const float *actual, const double *expected, size_t len,
                double atol, double rtol, or_check *result) {
    memset(result, 0, sizeof(*result));
    result->elements = len;
    for (size_t i = 0; i < len; ++i) {
        const double a = (double)actual[i], e = expected[i];
        if (!isfinite(a) || !isfinite(e)) {
            result->status = 1;
            result->first_bad = i;
            return;
        }
        const double error = fabs(a - e);
        if (!(error <= atol + rtol * fabs(e))) {
            result->status = 2;
            result->first_bad = i;
            return;
        }
        if (error > result->max_abs_error) result->max_abs_error = error;
        const double rel = error / fmax(fabs(e), atol);
        if (rel > result->max_relative_error) result->max_relative_error = rel;
    }
}

void or_check_gemm(uint32_t m, uint32_t n, uint32_t k, const float *a,
                   const float *b, const float *out, size_t budget, int fp16,
                   or_validation *result) {
    memset(result, 0, sizeof(*result));
    const size_t total = (size_t)m * n;
    if (!budget) {
        result->status = 3;
        return;
    }
    for (size_t i = 0; i < total; ++i) {
        if (!isfinite(out[i])) {
            result->status = 1;
            result->first_bad = i;
            return;
        }
    }
    const size_t count = budget < total ? budget : total;
    result->checked_elements = count;
    const double eps32 = 1.1920928955078125e-07;
    for (size_t sample = 0; sample < count; ++sample) {
        const size_t idx = count <= 1 ? 0 : sample * (total - 1) / (count - 1);
        const size_t row = idx / n, col = idx % n;
        double expected = 0.0, sum_abs = 0.0;
        for (size_t inner = 0; inner < k; ++inner) {
            const double product = (double)a[row * k + inner] * (double)b[inner * n + col];
            expected += product;
            sum_abs += fabs(product);
        }
        const double error = fabs((double)out[idx] - expected);
        const double coefficient = fp16 ? 0.0012 : fmax((double)k * eps32 * 2.0, 2e-6);
        const double tolerance = 2e-5 + coefficient * sum_abs;
        if (error > result->max_abs_error) result->max_abs_error = error;
        if (error / tolerance > result->max_scaled_error)
            result->max_scaled_error = error / tolerance;
        if (!(error <= tolerance)) {
            result->status = 2;
            result->first_bad = idx;
            return;
        }
    }
}
