/*
 * CPU oracle for the cPDE hot path -- TEST INFRASTRUCTURE ONLY (see cpde_oracle.h).
 * Compiled with -ffp-contract=off so that products and sums round like the
 * reference CPU build (no fused multiply-add on the default x86-64 target).
 */
#include "cpde_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define MAXK 6
#define MAXPART 203 /* Bell(6) */

/* ------------------------------------------------------------------ schema helpers */
static int find_row(int R, int V, const int* table, const int* counts) {
    for (int r = 0; r < R; ++r) {
        int ok = 1;
        for (int v = 0; v < V && ok; ++v) ok = table[r * (V + 1) + 1 + v] == counts[v];
        if (ok) return r;
    }
    return -1;
}

static int binom(int a, int b) {
    if (b < 0 || b > a) return 0;
    int r = 1;
    for (int i = 1; i <= b; ++i) r = r * (a - b + i) / i;
    return r;
}

/* dTab/Crs exactly as cuda/cpde_engine.cuh:476-498 (element (j,i) there is [i*R+j] here). */
int orc_pair_tables(int R, int V, const int* table, int* dtab, int* crs) {
    int diff[32];
    if (V > 32) return -1;
    for (int i = 0; i < R; ++i)
        for (int j = 0; j < R; ++j) {
            int coefficient = 1, valid = 1;
            for (int v = 0; v < V; ++v) {
                int a = table[j * (V + 1) + 1 + v], b = table[i * (V + 1) + 1 + v];
                diff[v] = a - b;
                if (a < b) valid = 0;
                coefficient *= a >= b ? binom(a, b) : 0;
            }
            dtab[i * R + j] = valid ? find_row(R, V, table, diff) : -1;
            crs[i * R + j] = coefficient ? coefficient : -1;
        }
    return 0;
}

/* Set partitions of a row's direction list (the k directions x..x y..y ... in
 * variable order, cuda/cpde_engine.cuh:420-448).  Each block maps to the schema
 * row of its sub-multi-index.  Enumeration: restricted growth strings. */
typedef struct { int blocks; int rows[MAXK]; } part_t;
typedef struct { int order; int count; part_t parts[MAXPART]; } row_parts_t;

static void enum_parts(int k, const int* dirs, int R, int V, const int* table, int pos, int* rgs,
                       int maxlab, row_parts_t* out) {
    if (pos == k) {
        part_t* p = &out->parts[out->count++];
        p->blocks = maxlab + 1;
        for (int b = 0; b <= maxlab; ++b) {
            int counts[32] = {0};
            for (int q = 0; q < k; ++q)
                if (rgs[q] == b) counts[dirs[q]]++;
            p->rows[b] = find_row(R, V, table, counts);
        }
        return;
    }
    for (int lab = 0; lab <= maxlab + 1; ++lab) {
        rgs[pos] = lab;
        enum_parts(k, dirs, R, V, table, pos + 1, rgs, lab > maxlab ? lab : maxlab, out);
    }
}

static row_parts_t* build_parts(int R, int V, const int* table) {
    row_parts_t* rp = (row_parts_t*)calloc((size_t)R, sizeof(row_parts_t));
    for (int r = 0; r < R; ++r) {
        int dirs[MAXK], k = 0;
        for (int v = 0; v < V; ++v)
            for (int c = 0; c < table[r * (V + 1) + 1 + v]; ++c) dirs[k++] = v;
        rp[r].order = k;
        rp[r].count = 0;
        if (k > 0) {
            int rgs[MAXK];
            rgs[0] = 0;
            enum_parts(k, dirs, R, V, table, 1, rgs, 0, &rp[r]);
        }
    }
    return rp;
}

static int check_schema(int R, int V, const int* table) {
    if (R <= 0 || V <= 0 || V > 26) return -1;
    if (table[0] != 0) return -1;
    for (int r = 0; r < R; ++r) {
        int s = 0;
        for (int v = 0; v < V; ++v) s += table[r * (V + 1) + 1 + v];
        if (s != table[r * (V + 1)] || s > MAXK) return -1;
    }
    return 0;
}

/* sigma^{(k)}, k=1..7, from q = 1/(1+e^z) (cuda/derivative_kernels_v4.cu:1-10,462-468). */
static void sigma_derivs(float z, float* s) {
    float q = 1.0f / (1.0f + expf(z));
    s[1] = q * (1.0f - q);
    s[2] = -s[1] * (1.0f - 2.0f * q);
    s[3] = s[1] * (1.0f - 6.0f * s[1]);
    s[4] = s[2] * (1.0f - 12.0f * s[1]);
    s[5] = s[1] - (5.0f * s[2]) * (6.0f * s[2]);
    s[6] = s[2] + 5.0f * (s[4] - s[2]) * (1.0f - 6.0f * s[1]);
    s[7] = (5.0f * s[1]) * (0.2f - (8.4f * s[1]) * (3.0f - 4.0f * (5.0f * s[1] + 5.0f * s[3])));
}

/* Partition sums M_m = sum over partitions with m blocks of prod z_B; result
 * sum_m s[m+shift] M_m accumulated left to right (shift 0: forward, 1: d^beta sigma'). */
static float partition_sum(const row_parts_t* rp, const float* z, long count, long e, const float* s, int shift) {
    float M[MAXK + 1] = {0};
    for (int t = 0; t < rp->count; ++t) {
        const part_t* p = &rp->parts[t];
        float prod = z[(long)p->rows[0] * count + e];
        for (int b = 1; b < p->blocks; ++b) prod = prod * z[(long)p->rows[b] * count + e];
        M[p->blocks] += prod;
    }
    float acc = s[1 + shift] * M[1];
    for (int m = 2; m <= rp->order; ++m) acc = acc + s[m + shift] * M[m];
    return acc;
}

int orc_compose(int R, int V, const int* table, long count, const float* z, float* y) {
    if (check_schema(R, V, table)) return -1;
    row_parts_t* rp = build_parts(R, V, table);
    for (long e = 0; e < count; ++e) {
        float s[8];
        float z0 = z[e];
        sigma_derivs(z0, s);
        y[e] = 1.0f / (1.0f + expf(-z0)); /* value row (cuda/derivative_kernels_v4.cu:742) */
        for (int r = 1; r < R; ++r) y[(long)r * count + e] = partition_sum(&rp[r], z, count, e, s, 0);
    }
    free(rp);
    return 0;
}

/* Jet of sigma'(z): u[0] = sigma'(z0), u[r] = d^{alpha_r} sigma'(z(x)) -- the
 * reference's DPlus rows (cuda/derivative_kernels_v4.cu:12-380, the shift-1
 * partition sums), here for every row. */
int orc_compose_prime(int R, int V, const int* table, long count, const float* z, float* u) {
    if (check_schema(R, V, table)) return -1;
    row_parts_t* rp = build_parts(R, V, table);
    for (long e = 0; e < count; ++e) {
        float s[8];
        sigma_derivs(z[e], s);
        u[e] = s[1];
        for (int r = 1; r < R; ++r) u[(long)r * count + e] = partition_sum(&rp[r], z, count, e, s, 1);
    }
    free(rp);
    return 0;
}

/* back_step (cuda/derivative_kernels_v4.cu:349-380): ascending i, in place, so each
 * g_j (j>i) is still the incoming dE/dy_j.  DPlus depends only on the difference
 * row, so it is evaluated once per row and element (identical floats). */
int orc_compose_adjoint(int R, int V, const int* table, long count, const float* z, float* g) {
    if (check_schema(R, V, table)) return -1;
    row_parts_t* rp = build_parts(R, V, table);
    int* dtab = (int*)malloc(sizeof(int) * (size_t)R * R);
    int* crs = (int*)malloc(sizeof(int) * (size_t)R * R);
    float* dplus = (float*)malloc(sizeof(float) * (size_t)R);
    orc_pair_tables(R, V, table, dtab, crs);
    for (long e = 0; e < count; ++e) {
        float s[8];
        sigma_derivs(z[e], s);
        dplus[0] = 0.0f;
        for (int r = 1; r < R; ++r) dplus[r] = partition_sum(&rp[r], z, count, e, s, 1);
        for (int i = 0; i < R; ++i) {
            float* ts = &g[(long)i * count + e];
            *ts *= s[1];
            for (int j = i + 1; j < R; ++j) {
                int dn = dtab[i * R + j];
                if (dn != -1) *ts += ((float)crs[i * R + j]) * g[(long)j * count + e] * dplus[dn];
            }
        }
    }
    free(rp);
    free(dtab);
    free(crs);
    free(dplus);
    return 0;
}

/* Portable serial column-major SGEMM (cpu/include/cublas_v2.h:34-40). ta/tb: 0 = N, 1 = T. */
void orc_gemm(int ta, int tb, int m, int n, int k, float alpha, const float* a, int lda,
              const float* b, int ldb, float beta, float* c, int ldc) {
    for (int j = 0; j < n; ++j)
        for (int i = 0; i < m; ++i) {
            float sum = 0;
            if (alpha != 0)
                for (int q = 0; q < k; ++q)
                    sum += (ta == 0 ? a[(long)q * lda + i] : a[(long)i * lda + q]) *
                           (tb == 0 ? b[(long)j * ldb + q] : b[(long)q * ldb + j]);
            c[(long)j * ldc + i] = alpha * sum + (beta == 0 ? 0 : beta * c[(long)j * ldc + i]);
        }
}

/* Sger with alpha=1, x=bias, y=ones over the first n columns (cpu/include/cublas_v2.h:51-53). */
static void add_bias(int m, int n, const float* bias, float* a, int lda) {
    for (int j = 0; j < n; ++j)
        for (int i = 0; i < m; ++i) a[(long)j * lda + i] += 1.0f * bias[i] * 1.0f;
}

/* Sgemv N with x=ones (cpu/include/cublas_v2.h:64-71). */
static void bias_gradient(int m, int n, const float* a, int lda, float beta, float* y) {
    for (int i = 0; i < m; ++i) {
        float sum = 0;
        for (int j = 0; j < n; ++j) sum += a[(long)j * lda + i] * 1.0f;
        y[i] = 1.0f * sum + (beta == 0 ? 0 : beta * y[i]);
    }
}

double orc_matching(int R, int outputs, int width, int valid, int offset, int samples,
                    const float* y, float* g, const float* target, const int* target_rows,
                    const float* weights, int weight_samples, int gradient,
                    int* bad_sample, int* bad_component) {
    double loss = 0;
    int bs = 0x7fffffff, bc = 0x7fffffff;
    for (int p = 0; p < width; ++p) {
        float value = 0.0f;
        for (int d = 0; d < R; ++d)
            for (int o = 0; o < outputs; ++o) {
                long i = (long)d * width * outputs + (long)p * outputs + o;
                if (gradient) g[i] = 0.0f;
                if (p >= valid) continue;
                int wp = weight_samples == 1 ? 0 : offset + p;
                float w = weights[((long)d * weight_samples + wp) * outputs + o];
                if (w == 0.0f) continue;
                float r = y[i] - target[(long)target_rows[d] * samples * outputs + (long)(offset + p) * outputs + o];
                value += w * r * r;
                if (gradient) g[i] = 2.0f * w * r;
            }
        if (!isfinite(value) && (offset + p < bs || (offset + p == bs && -1 < bc))) { bs = offset + p; bc = -1; }
        loss += (double)value;
        if (gradient && p < valid)
            for (int d = 0; d < R; ++d)
                for (int o = 0; o < outputs; ++o) {
                    long i = (long)d * width * outputs + (long)p * outputs + o;
                    int comp = d * outputs + o;
                    if (!isfinite(g[i]) && (offset + p < bs || (offset + p == bs && comp < bc))) { bs = offset + p; bc = comp; }
                }
    }
    if (bad_sample) *bad_sample = bs;
    if (bad_component) *bad_component = bc;
    return loss;
}

/* ------------------------------------------------------------------ network */
typedef struct {
    int L;
    const int* neurons;
    const int* linear;
    int R, V, w;
    const int* table;
    float** z; /* z[l]: [R][w][n_l]; z[0] is the input stack */
    float** g; /* g[l]: adjoint of z[l] */
    float* y;  /* activation scratch, max n */
} net_t;

static const float* activation(net_t* N, int l) {
    if (N->linear[l]) return N->z[l];
    orc_compose(N->R, N->V, N->table, (long)N->neurons[l] * N->w, N->z[l], N->y);
    return N->y;
}

/* network::feedforward (cuda/cpde_engine.cuh:889-913). */
static void net_forward(net_t* N, const float* const* W) {
    for (int t = 0; t + 1 < N->L; ++t) {
        int ni = N->neurons[t], no = N->neurons[t + 1];
        const float* Y = activation(N, t);
        orc_gemm(0, 0, no, N->R * N->w, ni, 1.0f, W[t], no, Y, ni, 0.0f, N->z[t + 1], no);
        add_bias(no, N->w, W[t] + (long)no * ni, N->z[t + 1], no);
    }
}

/* network::backprop (cuda/cpde_engine.cuh:947-991). */
static void net_backward(net_t* N, const float* const* W, float* const* grad, float beta) {
    for (int t = N->L - 2; t >= 0; --t) {
        int ni = N->neurons[t], no = N->neurons[t + 1];
        bias_gradient(no, N->w, N->g[t + 1], no, beta, grad[t] + (long)no * ni);
        if (t > 0) {
            orc_gemm(1, 0, ni, N->R * N->w, no, 1.0f, W[t], no, N->g[t + 1], no, 0.0f, N->g[t], ni);
            if (!N->linear[t]) orc_compose_adjoint(N->R, N->V, N->table, (long)ni * N->w, N->z[t], N->g[t]);
        }
        const float* Y = activation(N, t);
        orc_gemm(0, 1, no, ni, N->R * N->w, 1.0f, N->g[t + 1], no, Y, ni, beta, grad[t], no);
    }
}

static int net_alloc(net_t* N, int L, const int* neurons, const int* linear, int R, int V, const int* table, int w) {
    N->L = L; N->neurons = neurons; N->linear = linear; N->R = R; N->V = V; N->table = table; N->w = w;
    N->z = (float**)calloc((size_t)L, sizeof(float*));
    N->g = (float**)calloc((size_t)L, sizeof(float*));
    int nmax = 0;
    for (int l = 0; l < L; ++l) {
        N->z[l] = (float*)calloc((size_t)R * w * neurons[l], sizeof(float));
        N->g[l] = (float*)calloc((size_t)R * w * neurons[l], sizeof(float));
        if (neurons[l] > nmax) nmax = neurons[l];
    }
    N->y = (float*)calloc((size_t)R * w * nmax, sizeof(float));
    return 0;
}

static void net_free(net_t* N) {
    for (int l = 0; l < N->L; ++l) { free(N->z[l]); free(N->g[l]); }
    free(N->z); free(N->g); free(N->y);
}

int orc_forward(int L, const int* neurons, const int* linear, const float* const* W,
                int R, int V, const int* table, int w, const float* x, float* out) {
    if (check_schema(R, V, table)) return -1;
    net_t N;
    net_alloc(&N, L, neurons, linear, R, V, table, w);
    memcpy(N.z[0], x, sizeof(float) * (size_t)R * w * neurons[0]);
    net_forward(&N, W);
    memcpy(out, N.z[L - 1], sizeof(float) * (size_t)R * w * neurons[L - 1]);
    net_free(&N);
    return 0;
}

/* Server::pass for one matching cost (cuda/cpde_server.cu:223-257): chunk loop,
 * activate with zero padding (:158-170), forward, cost, backward with beta 0 on
 * the first chunk and 1 afterwards. */
double orc_matching_epoch(int L, const int* neurons, const int* linear, const float* const* W,
                          float* const* grad, int R, int V, const int* table, int samples, int chunk,
                          const float* x, int data_rows, const int* rows, const float* target,
                          const int* target_rows, const float* weights, int weight_samples,
                          float* outputs) {
    (void)data_rows;
    if (check_schema(R, V, table)) return NAN;
    int width = chunk && chunk < samples ? chunk : samples;
    int n0 = neurons[0], no = neurons[L - 1];
    net_t N;
    net_alloc(&N, L, neurons, linear, R, V, table, width);
    double loss = 0;
    int first = 1;
    for (int offset = 0; offset < samples; offset += width) {
        int valid = samples - offset < width ? samples - offset : width;
        for (int d = 0; d < R; ++d) {
            float* dest = N.z[0] + (long)d * width * n0;
            memcpy(dest, x + (long)rows[d] * samples * n0 + (long)offset * n0, sizeof(float) * (size_t)valid * n0);
            if (valid < width) memset(dest + (long)valid * n0, 0, sizeof(float) * (size_t)(width - valid) * n0);
        }
        net_forward(&N, W);
        int bs, bc;
        loss += orc_matching(R, no, width, valid, offset, samples, N.z[L - 1], N.g[L - 1], target, target_rows,
                             weights, weight_samples, 1, &bs, &bc);
        if (outputs)
            for (int d = 0; d < R; ++d)
                memcpy(outputs + (long)d * samples * no + (long)offset * no, N.z[L - 1] + (long)d * width * no,
                       sizeof(float) * (size_t)valid * no);
        net_backward(&N, W, grad, first ? 0.0f : 1.0f);
        first = 0;
    }
    net_free(&N);
    return loss;
}

/* gradient_blocks semantics (cuda/reduction_kernels.cuh:81-98): promote before squaring. */
orc_grad_stats_t orc_gradient_stats(const float* g, int count) {
    orc_grad_stats_t s = {0.0, 0.0, 0ull, 0x7fffffff};
    for (int i = 0; i < count; ++i) {
        double v = g[i];
        if (!isfinite(v)) {
            s.nonfinite++;
            if (i < s.first) s.first = i;
        } else {
            s.squared_norm += v * v;
            double m = fabs(v);
            if (m > s.max_abs) s.max_abs = m;
        }
    }
    return s;
}

/* Resile_k (cuda/derivative_kernels_v4.cu:752-778), float products as there. */
void orc_rprop(int count, float* W, float* step, float* ga, float* gi) {
    for (int t = 0; t < count; ++t) {
        if (ga[t] * gi[t] > 0) step[t] *= 1.2f;
        float nW = W[t] - copysignf(step[t], ga[t]);
        if (ga[t] * gi[t] < 0) {
            W[t] += copysignf(step[t], gi[t]);
            step[t] *= 0.5f;
            ga[t] = 0.0f;
        } else if (ga[t] != 0.0f) {
            if (fabsf(nW) <= 20.0f) W[t] = nW;
            else { step[t] = 0.1f; ga[t] = 0.0f; }
        }
    }
}

/* Reset_Resile_k (cuda/derivative_kernels_v4.cu:801-814). */
void orc_restore_steps(int count, float floor_step, float* step, float* ga, float* gi) {
    for (int t = 0; t < count; ++t)
        if (step[t] < floor_step) { step[t] = floor_step; ga[t] = 0.0f; gi[t] = 0.0f; }
}

/* Set_Resile_k (cuda/derivative_kernels_v4.cu:825-832). */
void orc_set_steps(int count, float value, float* step, float* ga, float* gi) {
    for (int t = 0; t < count; ++t) { step[t] = value; ga[t] = gi[t] = 0.0f; }
}

/* ADAM_k (cuda/derivative_kernels_v4.cu:780-799); the epsilon is a double literal there. */
void orc_adam(int count, float* W, const float* g, float* m, float* v, float lr, float beta1, float beta2,
              float beta1t, float beta2t) {
    for (int t = 0; t < count; ++t) {
        m[t] = beta1 * m[t] + (1 - beta1) * g[t];
        v[t] = beta2 * v[t] + (1 - beta2) * g[t] * g[t];
        float mh = m[t] / (1 - beta1t), vh = v[t] / (1 - beta2t);
        float nW = (float)(W[t] - lr * mh / (sqrtf(vh) + 1e-8));
        if (fabsf(nW) <= 20.0f) W[t] = nW;
    }
}
