/*
 * CPU oracle for the cPDE hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the oracle for the MI355X kernels.  Only tests/, the package's
 * smoke() and bench.py's cpu_baseline leg may load it; the product path never
 * links, calls or falls back to it.
 *
 * It restates the reference's arithmetic in plain C, fp32 like the reference:
 *   - derivative schema tables          cuda/cpde_engine.cuh:391-498
 *   - forward sigmoid composition        cuda/derivative_kernels_v4.cu:382-745
 *   - sigma' composition (DPlus rows)    cuda/derivative_kernels_v4.cu:12-380
 *   - adjoint composition (back_step)    cuda/derivative_kernels_v4.cu:12-380
 *   - serial column-major BLAS order     cpu/include/cublas_v2.h:34-40,51-53,64-71
 *   - network forward / backward         cuda/cpde_engine.cuh:889-913,947-991
 *   - matching cost                      cuda/cost_kernels.cuh:6-35
 *   - gradient statistics                cuda/reduction_kernels.cuh:81-98
 *   - RPROP / step set / step restore    cuda/derivative_kernels_v4.cu:752-832
 *   - Adam                               cuda/derivative_kernels_v4.cu:780-799
 *
 * Layouts are the reference's: a stack is [row][point][neuron] (neuron fastest);
 * schema tables are row-major rows x (variables+1) = (order, counts...);
 * a weight block is n_out x (n_in+1) column-major with the bias as last column.
 *
 * Pinning (which check covers which function) is listed in the tests under
 * tests/test_oracle_*.py; every function here is pinned by at least one of:
 * reference-server golden vectors, published known answers, a Taylor-jet
 * composition in float64, finite differences, or a textbook float64 product.
 */
#ifndef CPDE_ORACLE_H
#define CPDE_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Row index of alpha_j - alpha_i (or -1) and C(alpha_j, alpha_i), stored at [i*R+j]. */
int orc_pair_tables(int R, int V, const int* table, int* dtab, int* crs);

/* y[r][e] = d^{alpha_r} sigma(z)[e] for count independent elements. */
int orc_compose(int R, int V, const int* table, long count, const float* z, float* y);
/* u[r][e] = d^{alpha_r} sigma'(z)[e]: the jet of sigma' the adjoint contracts with. */
int orc_compose_prime(int R, int V, const int* table, long count, const float* z, float* u);
/* In place: g holds dE/dy on entry and dE/dz on exit. */
int orc_compose_adjoint(int R, int V, const int* table, long count, const float* z, float* g);

void orc_gemm(int ta, int tb, int m, int n, int k, float alpha, const float* a, int lda,
              const float* b, int ldb, float beta, float* c, int ldc);

/* Matching cost over one chunk (cuda/cost_kernels.cuh:6-35).  y, g: [R][width][outputs];
 * target: [target_rows_total][samples][outputs]; weights: [R][weight_samples][outputs].
 * Returns the double loss; *bad_sample / *bad_component get the first bad location. */
double orc_matching(int R, int outputs, int width, int valid, int offset, int samples,
                    const float* y, float* g, const float* target, const int* target_rows,
                    const float* weights, int weight_samples, int gradient,
                    int* bad_sample, int* bad_component);

/* One epoch of one matching cost over all chunks: forward, cost, backward.
 * x: input data [Rd][samples][n0] with rows selected by rows[R]; target as above.
 * W[t]: n_{t+1} x (n_t+1); grad[t] receives the gradient (overwritten on the
 * first chunk, accumulated afterwards, cuda/cpde_server.cu:255).
 * outputs (optional): [R][samples][n_out].  Returns the loss. */
double orc_matching_epoch(int L, const int* neurons, const int* linear, const float* const* W,
                          float* const* grad, int R, int V, const int* table, int samples, int chunk,
                          const float* x, int data_rows, const int* rows, const float* target,
                          const int* target_rows, const float* weights, int weight_samples,
                          float* outputs);

/* Forward only, one chunk of width w (no padding): x [R][w][n0] -> out [R][w][n_out]. */
int orc_forward(int L, const int* neurons, const int* linear, const float* const* W,
                int R, int V, const int* table, int w, const float* x, float* out);

typedef struct { double squared_norm, max_abs; unsigned long long nonfinite; int first; } orc_grad_stats_t;
orc_grad_stats_t orc_gradient_stats(const float* g, int count);

void orc_rprop(int count, float* W, float* step, float* g_active, float* g_inactive);
void orc_restore_steps(int count, float floor_step, float* step, float* g_active, float* g_inactive);
void orc_set_steps(int count, float value, float* step, float* g_active, float* g_inactive);
void orc_adam(int count, float* W, const float* g, float* m, float* v, float lr, float beta1, float beta2,
              float beta1t, float beta2t);

#ifdef __cplusplus
}
#endif
#endif
