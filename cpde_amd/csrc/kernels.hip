// gfx950 kernels of the cPDE hot path.
//
// Stacks are [point][row][neuron] (neuron fastest): one GEMM column is one
// (point,row) pair, so a point's derivative rows are adjacent columns.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "common.hpp"

namespace cpde {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// sigma^{(k)}(z), k = 1..7, from q = 1/(1+e^z): the reference's recurrences
// (cuda/derivative_kernels_v4.cu:1-10, 462-468; KNOWN_ISSUES F04 keeps the tails).
__device__ __forceinline__ void sigma_derivatives(float z, float* s) {
    const float q = 1.0f / (1.0f + expf(z));
    s[1] = q * (1.0f - q);
    s[2] = -s[1] * (1.0f - 2.0f * q);
    s[3] = s[1] * (1.0f - 6.0f * s[1]);
    s[4] = s[2] * (1.0f - 12.0f * s[1]);
    s[5] = s[1] - (5.0f * s[2]) * (6.0f * s[2]);
    s[6] = s[2] + 5.0f * (s[4] - s[2]) * (1.0f - 6.0f * s[1]);
    s[7] = (5.0f * s[1]) * (0.2f - (8.4f * s[1]) * (3.0f - 4.0f * (5.0f * s[1] + 5.0f * s[3])));
}

// Sum over a row's multiset-partition terms: sum_m s[m+shift] * M_m, with
// M_m = sum_terms coefficient * prod(block rows).  `col` is this lane's private
// LDS column (stride B floats per row); `pos` walks the uniform term table.
template <int B, int SHIFT>
__device__ __forceinline__ float partition_sum(const float* col, const int* __restrict__ words, int& pos,
                                               const float* s) {
    const int k = words[pos++];
    float acc = 0.0f;
#pragma unroll
    for (int m = 1; m <= kMaxOrder; ++m) {
        if (m <= k) {
            const int count = words[pos++];
            float M = 0.0f;
            for (int q = 0; q < count; ++q) {
                const float c = __int_as_float(words[pos]);
                const unsigned w0 = unsigned(words[pos + 1]), w1 = unsigned(words[pos + 2]);
                pos += 3;
                float prod = col[(w0 & 255u) * B];
                if (m > 1) prod *= col[((w0 >> 8) & 255u) * B];
                if (m > 2) prod *= col[((w0 >> 16) & 255u) * B];
                if (m > 3) prod *= col[(w0 >> 24) * B];
                if (m > 4) prod *= col[(w1 & 255u) * B];
                if (m > 5) prod *= col[((w1 >> 8) & 255u) * B];
                M = fmaf(c, prod, M);
            }
            acc = (m == 1) ? s[1 + SHIFT] * M : fmaf(s[m + SHIFT], M, acc);
        }
    }
    return acc;
}

// Forward composition y = d^alpha sigma(z) for every row of one (point, neuron)
// per lane (replaces d0..d6, cuda/derivative_kernels_v4.cu:382-745, and the
// per-row launch loop network::D, cuda/cpde_engine.cuh:852-866).
template <int B>
__global__ __launch_bounds__(B) void compose_forward_kernel(const float* __restrict__ z, float* __restrict__ y, int R,
                                                            int n, int elements, const int* __restrict__ words) {
    extern __shared__ float lds[];
    const int t = threadIdx.x;
    const int e = blockIdx.x * B + t;
    const bool live = e < elements;
    const int p = live ? e / n : 0, i = live ? e - p * n : 0;
    const size_t base = size_t(p) * R * n + i;
    float* col = lds + t;
    for (int r = 0; r < R; ++r) col[r * B] = live ? z[base + size_t(r) * n] : 0.0f;
    float s[8];
    const float z0 = col[0];
    sigma_derivatives(z0, s);
    if (live) y[base] = 1.0f / (1.0f + expf(-z0));
    int pos = 0;
    for (int r = 1; r < R; ++r) {
        const float v = partition_sum<B, 0>(col, words, pos, s);
        if (live) y[base + size_t(r) * n] = v;
    }
}

// Adjoint composition (replaces back_step + DPlus/d1p..d6p,
// cuda/derivative_kernels_v4.cu:12-380):
//   g_z[i] = sigma'(z) g_y[i] + sum_{j>i, alpha_j>=alpha_i} C(alpha_j,alpha_i) g_y[j] D[alpha_j-alpha_i]
// with D[beta] = d^beta sigma'(z) evaluated once per row (it depends only on the
// difference row), computed in place over the z column in descending row order.
template <int B>
__global__ __launch_bounds__(B) void compose_adjoint_kernel(const float* __restrict__ z, float* __restrict__ g, int R,
                                                            int n, int elements, const int* __restrict__ words,
                                                            const int* __restrict__ fwd_offset, int pair_begin) {
    extern __shared__ float lds[];
    const int t = threadIdx.x;
    const int e = blockIdx.x * B + t;
    const bool live = e < elements;
    const int p = live ? e / n : 0, i = live ? e - p * n : 0;
    const size_t base = size_t(p) * R * n + i;
    float* zc = lds + t;
    float* gc = lds + size_t(R) * B + t;
    for (int r = 0; r < R; ++r) {
        zc[r * B] = live ? z[base + size_t(r) * n] : 0.0f;
        gc[r * B] = live ? g[base + size_t(r) * n] : 0.0f;
    }
    float s[8];
    sigma_derivatives(zc[0], s);
    for (int r = R - 1; r >= 1; --r) {
        int pos = fwd_offset[r];
        const float d = partition_sum<B, 1>(zc, words, pos, s);
        zc[r * B] = d;
    }
    int pos = pair_begin;
    for (int a = 0; a < R; ++a) {
        const int count = words[pos++];
        float acc = s[1] * gc[a * B];
        for (int q = 0; q < count; ++q) {
            const int j = words[pos], dn = words[pos + 1];
            const float c = __int_as_float(words[pos + 2]);
            pos += 3;
            acc = acc + (c * gc[j * B]) * zc[dn * B];
        }
        if (live) g[base + size_t(a) * n] = acc;
    }
}

static int compose_block(int R, int arrays) {
    // Largest block (256/128/64) whose private columns fit in 64 KB of LDS.
    for (int b = 256; b >= 64; b /= 2)
        if (size_t(arrays) * R * b * sizeof(float) <= 65536) return b;
    return 64;
}

void launch_compose_forward(Device& d, const Plan& p, const float* z, float* y, int n) {
    const int R = p.rows, elements = p.width * n;
    const int b = compose_block(R, 1);
    const size_t lds = size_t(R) * b * sizeof(float);
    const int grid = (elements + b - 1) / b;
    TraceScope trace(d, kTraceComposeForward, 8.0 * double(elements) * R);  // read z, write y
    if (b == 256)
        hipLaunchKernelGGL(compose_forward_kernel<256>, grid, 256, lds, d.stream, z, y, R, n, elements, p.dev_tables);
    else if (b == 128)
        hipLaunchKernelGGL(compose_forward_kernel<128>, grid, 128, lds, d.stream, z, y, R, n, elements, p.dev_tables);
    else
        hipLaunchKernelGGL(compose_forward_kernel<64>, grid, 64, lds, d.stream, z, y, R, n, elements, p.dev_tables);
    HIP_CHECK(hipGetLastError());
}

void launch_compose_adjoint(Device& d, const Plan& p, const float* z, float* g, int n) {
    const int R = p.rows, elements = p.width * n;
    const int b = compose_block(R, 2);
    const size_t lds = 2 * size_t(R) * b * sizeof(float);
    const int grid = (elements + b - 1) / b;
    const int* offsets = p.dev_tables + p.tables.words.size();
    TraceScope trace(d, kTraceComposeAdjoint, 12.0 * double(elements) * R);  // read z and g_y, write g_z
    const int pair_begin = p.tables.pair_offset[0];
    if (b == 256)
        hipLaunchKernelGGL(compose_adjoint_kernel<256>, grid, 256, lds, d.stream, z, g, R, n, elements, p.dev_tables,
                           offsets, pair_begin);
    else if (b == 128)
        hipLaunchKernelGGL(compose_adjoint_kernel<128>, grid, 128, lds, d.stream, z, g, R, n, elements, p.dev_tables,
                           offsets, pair_begin);
    else
        hipLaunchKernelGGL(compose_adjoint_kernel<64>, grid, 64, lds, d.stream, z, g, R, n, elements, p.dev_tables,
                           offsets, pair_begin);
    HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------------------------------
// FP32 MFMA GEMM: C[M x N] = A[M x K] * B[K x N] on v_mfma_f32_32x32x2_f32 (true
// fp32, no reduced-precision shortcut).  256 lanes = WM x WN waves; each wave owns
// a (BM/WM) x (BN/WN) tile made of 32x32 MFMA blocks.  Tiles of A and B pass
// through LDS in K chunks of BK.  Split-K: blockIdx.z takes K range
// [z*k_split, (z+1)*k_split) and writes its partial product to C + z*ldc*N.
constexpr int BK = 16;

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_kernel(int M, int N, int K, const float* __restrict__ A, int lda, int a_t,
                                                   const float* __restrict__ Bm, int ldb, int b_t, float* __restrict__ C,
                                                   int ldc, const float* __restrict__ bias, int period, int k_split) {
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int IM = TM / 32, IN = TN / 32;
    __shared__ float As[BK][BM + 1];
    __shared__ float Bs[BK][BN + 1];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    int kbegin = 0, kend = K;
    if (k_split > 0) {
        kbegin = blockIdx.z * k_split;
        kend = min(K, kbegin + k_split);
        C += size_t(blockIdx.z) * ldc * N;
    }
    floatx16 acc[IM][IN];
#pragma unroll
    for (int a = 0; a < IM; ++a)
#pragma unroll
        for (int b = 0; b < IN; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    for (int k0 = kbegin; k0 < kend; k0 += BK) {
        // A tile -> As[k][m]
#pragma unroll
        for (int idx = t; idx < BM * BK; idx += 256) {
            int m, k;
            if (a_t) { k = idx % BK; m = idx / BK; }
            else { m = idx % BM; k = idx / BM; }
            const int gm = m0 + m, gk = k0 + k;
            float v = 0.0f;
            if (gm < M && gk < kend) v = a_t ? A[gk + size_t(lda) * gm] : A[gm + size_t(lda) * gk];
            As[k][m] = v;
        }
        // B tile -> Bs[k][n]
#pragma unroll
        for (int idx = t; idx < BN * BK; idx += 256) {
            int n, k;
            if (b_t) { n = idx % BN; k = idx / BN; }
            else { k = idx % BK; n = idx / BK; }
            const int gn = n0 + n, gk = k0 + k;
            float v = 0.0f;
            if (gn < N && gk < kend) v = b_t ? Bm[gn + size_t(ldb) * gk] : Bm[gk + size_t(ldb) * gn];
            Bs[k][n] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            const int kr = kk + (lane >> 5), lc = lane & 31;
            float av[IM], bv[IN];
#pragma unroll
            for (int a = 0; a < IM; ++a) av[a] = As[kr][wm * TM + a * 32 + lc];
#pragma unroll
            for (int b = 0; b < IN; ++b) bv[b] = Bs[kr][wn * TN + b * 32 + lc];
#pragma unroll
            for (int a = 0; a < IM; ++a)
#pragma unroll
                for (int b = 0; b < IN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    // Accumulator layout of a 32x32 block: lane l, register v holds
    // row 8*(v/4) + 4*(l/32) + v%4, column l%32.
#pragma unroll
    for (int a = 0; a < IM; ++a)
#pragma unroll
        for (int b = 0; b < IN; ++b) {
            const int gn = n0 + wn * TN + b * 32 + (lane & 31);
            if (gn >= N) continue;
            const bool add_bias = bias != nullptr && (gn % period) == 0;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int gm = m0 + wm * TM + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (gm < M) C[gm + size_t(ldc) * gn] = acc[a][b][v] + (add_bias ? bias[gm] : 0.0f);
            }
        }
}

static void gemm_dispatch(Device& d, int M, int N, int K, const float* A, int lda, bool a_t, const float* B, int ldb,
                          bool b_t, float* C, int ldc, const float* bias, int period, int splits, int k_split) {
    if (M <= 32) {
        dim3 grid((M + 31) / 32, (N + 127) / 128, splits);
        hipLaunchKernelGGL((gemm_kernel<32, 128, 1, 4>), grid, 256, 0, d.stream, M, N, K, A, lda, int(a_t), B, ldb,
                           int(b_t), C, ldc, bias, period, k_split);
    } else {
        dim3 grid((M + 127) / 128, (N + 63) / 64, splits);
        hipLaunchKernelGGL((gemm_kernel<128, 64, 4, 1>), grid, 256, 0, d.stream, M, N, K, A, lda, int(a_t), B, ldb,
                           int(b_t), C, ldc, bias, period, k_split);
    }
    HIP_CHECK(hipGetLastError());
}

void launch_gemm(Device& d, int M, int N, int K, const float* A, int lda, bool a_t, const float* B, int ldb, bool b_t,
                 float* C, int ldc, const float* bias, int period) {
    if (M <= 0 || N <= 0) return;
    TraceScope trace(d, a_t ? kTraceGemmTransposed : kTraceGemm, 2.0 * M * double(N) * K);
    gemm_dispatch(d, M, N, K, A, lda, a_t, B, ldb, b_t, C, ldc, bias, period > 0 ? period : 1, 1, 0);
}

// ------------------------------------------------------------------------------------------
// Output transition with few outputs: z[col][o] = sum_i W[o + NO*i] y[col][i]
// (+ bias on value-row columns).  One wave per column, lanes stride the inputs,
// fixed-order wave reduction.
__global__ __launch_bounds__(256) void output_forward_kernel(const float* __restrict__ W, const float* __restrict__ Y,
                                                             float* __restrict__ Z, int NI, int NO, int R,
                                                             int columns) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int col = blockIdx.x * 4 + wave; col < columns; col += gridDim.x * 4) {
        const float* y = Y + size_t(col) * NI;
        for (int o = 0; o < NO; ++o) {
            float s = 0.0f;
            for (int i = lane; i < NI; i += 64) s = fmaf(W[o + NO * i], y[i], s);
            for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
            if (lane == 0) Z[size_t(col) * NO + o] = s + ((col % R) == 0 ? W[o + NO * NI] : 0.0f);
        }
    }
}

void launch_output_forward(Device& d, const float* W, const float* Y, float* Z, int NI, int NO, int R, int columns) {
    TraceScope trace(d, kTraceGemm, 2.0 * NI * NO * double(columns));
    const int blocks = std::max(1, std::min(4096, (columns + 3) / 4));
    hipLaunchKernelGGL(output_forward_kernel, blocks, 256, 0, d.stream, W, Y, Z, NI, NO, R, columns);
    HIP_CHECK(hipGetLastError());
}

// Weight gradients of several transitions in one launch: dW_t = G_t Y_t^T over
// K = R*width columns, split over K into fixed ranges; each block writes its
// split's partial row-major [m][N+1] (entry N: the bias gradient, the sum over
// value-row columns), reduced in split order by reduce_grouped_kernel so the
// result does not depend on scheduling.  Two block roles:
//  * matrix-core tiles (M, N > 16): a 128x128 (or 64x64) tile, K staged
//    through LDS in chunks of 32 columns (double-buffered, the next chunk's
//    global loads in flight during the current chunk's MFMAs);
//  * thin transitions (M or N <= 16: the input and output layers): lanes
//    stride the wide side and accumulate the narrow side in registers.
constexpr int kWgKC = kWgradChunk;                 // columns per LDS chunk
constexpr int kWgLds = 2 * 2 * kWgKC * (128 + 4);  // floats of LDS shared by the block roles

// Matrix-core tile of one split: TILE x TILE of dW (TILE = 128, or 64 for
// transitions no wider than 64), wave = quadrant of (TILE/64)^2 MFMA 32x32
// blocks (per k-step: TILE/64 A + TILE/64 B operands feed (TILE/64)^2 MFMAs).
template <int TILE>
__device__ __forceinline__ void wgrad_tile(const WgradArgs& a, int t, int local, float* lds) {
    constexpr int LD = TILE + 4;    // LDS row stride of a chunk
    constexpr int WX = TILE / 64;   // MFMA blocks per wave and dimension
    constexpr int RP = 1024 / TILE; // staged rows per pass (256 threads x float4)
    constexpr int J = kWgKC / RP;   // passes per chunk
    typedef float Chunk[kWgKC][LD];
    Chunk* As = reinterpret_cast<Chunk*>(lds);
    Chunk* Bs = reinterpret_cast<Chunk*>(lds + 2 * kWgKC * LD);
    const int M = a.M[t], N = a.N[t], K = a.K[t];
    const int tiles_m = (M + TILE - 1) / TILE, tiles_n = (N + TILE - 1) / TILE;
    const int tile = local % (tiles_m * tiles_n), split = local / (tiles_m * tiles_n);
    const int m0 = (tile % tiles_m) * TILE, n0 = (tile / tiles_m) * TILE;
    const int kbegin = split * a.kchunk[t], kend = min(K, kbegin + a.kchunk[t]);
    const float* __restrict__ G = a.G[t];
    const float* __restrict__ Y = a.Y[t];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i = lane & 31, h = lane >> 5;
    // staging: thread -> 4 consecutive columns at 4*(tid % (TILE/4)) of rows tid/(TILE/4) + RP*j;
    // pointers advance by one chunk per step, bounds are per thread and fixed
    const int sc = 4 * (tid % (TILE / 4)), sr = tid / (TILE / 4);
    const bool g_vec = (M % 4) == 0 && m0 + sc + 3 < M, y_vec = (N % 4) == 0 && n0 + sc + 3 < N;
    const int g_cols = max(0, min(4, M - m0 - sc)), y_cols = max(0, min(4, N - n0 - sc));
    const float* gp = G + size_t(kbegin + sr) * M + m0 + sc;
    const float* yp = Y + size_t(kbegin + sr) * N + n0 + sc;
    auto load = [](const float* p, bool vec, int cols) -> float4 {
        if (vec) return *reinterpret_cast<const float4*>(p);
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (cols > 0) v.x = p[0];
        if (cols > 1) v.y = p[1];
        if (cols > 2) v.z = p[2];
        if (cols > 3) v.w = p[3];
        return v;
    };
    auto stage = [&](float4* ga, float4* ya, int k0) {  // rows k0 + sr + RP*j of G and Y
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool in = k0 + sr + RP * j < kend;
            ga[j] = in ? load(gp + size_t(RP) * j * M, g_vec, g_cols) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            ya[j] = in ? load(yp + size_t(RP) * j * N, y_vec, y_cols) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        gp += size_t(kWgKC) * M;
        yp += size_t(kWgKC) * N;
    };
    floatx16 acc[WX][WX];
#pragma unroll
    for (int x = 0; x < WX; ++x)
#pragma unroll
        for (int y = 0; y < WX; ++y)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[x][y][v] = 0.0f;
    float bias = 0.0f;  // tile column 0 blocks: thread tid < TILE sums G[k][m0+tid] over value rows
    int value_col = (kbegin + a.R[t] - 1) / a.R[t] * a.R[t];  // next value-row column
    const int wm = (TILE / 2) * (wave & 1), wn = (TILE / 2) * (wave >> 1);
    float4 ga[J], ya[J];
    stage(ga, ya, kbegin);
    int buf = 0;
    for (int k0 = kbegin; k0 < kend; k0 += kWgKC) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            *reinterpret_cast<float4*>(&As[buf][sr + RP * j][sc]) = ga[j];
            *reinterpret_cast<float4*>(&Bs[buf][sr + RP * j][sc]) = ya[j];
        }
        __syncthreads();
        if (k0 + kWgKC < kend) stage(ga, ya, k0 + kWgKC);
        __builtin_amdgcn_iglp_opt(0);  // interleave the LDS operand reads with the MFMAs
#pragma unroll
        for (int kk = 0; kk < kWgKC; kk += 2) {
            float av[WX], bv[WX];
#pragma unroll
            for (int x = 0; x < WX; ++x) {
                av[x] = As[buf][kk + h][wm + 32 * x + i];
                bv[x] = Bs[buf][kk + h][wn + 32 * x + i];
            }
#pragma unroll
            for (int x = 0; x < WX; ++x)
#pragma unroll
                for (int y = 0; y < WX; ++y)
                    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[x], bv[y], acc[x][y], 0, 0, 0);
        }
        if (n0 == 0 && tid < TILE) {
            const int stop = min(kend, k0 + kWgKC);
            for (; value_col < stop; value_col += a.R[t]) bias += As[buf][value_col - k0][tid];
        }
        buf ^= 1;
    }
    float* P = a.partial[t] + size_t(split) * M * (N + 1);
#pragma unroll
    for (int x = 0; x < WX; ++x)
#pragma unroll
        for (int y = 0; y < WX; ++y)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int mrow = m0 + wm + 32 * x + 8 * (v >> 2) + 4 * h + (v & 3), ncol = n0 + wn + 32 * y + i;
                if (mrow < M && ncol < N) P[size_t(mrow) * (N + 1) + ncol] = acc[x][y][v];
            }
    if (n0 == 0 && tid < TILE && m0 + tid < M) P[size_t(m0 + tid) * (N + 1) + N] = bias;
}

__device__ __forceinline__ void wgrad_thin(const WgradArgs& a, int t, int split, float* red) {
    const int M = a.M[t], N = a.N[t], K = a.K[t], R = a.R[t];
    const int kbegin = split * a.kchunk[t], kend = min(K, kbegin + a.kchunk[t]);
    const float* __restrict__ G = a.G[t];
    const float* __restrict__ Y = a.Y[t];
    float* P = a.partial[t] + size_t(split) * M * (N + 1);
    const bool wide_m = N <= 16;  // otherwise M <= 16 and the wide side is n
    const int wide = wide_m ? M : N, narrow = wide_m ? N : M;
    const int Wc = min(wide, 256), S = 256 / Wc;
    const int s = threadIdx.x / Wc, w = threadIdx.x - s * Wc;
    for (int w0 = 0; w0 < wide; w0 += Wc) {
        const int wi = w0 + w;
        float acc[16], bias[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[q] = bias[q] = 0.0f;
        if (s < S && wi < wide) {
            int k = kbegin + s;
            for (; k + 3 * S < kend; k += 4 * S) {
                float wv[4], nv[4][16];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const size_t kk = size_t(k + u * S);
                    wv[u] = wide_m ? G[kk * M + wi] : Y[kk * N + wi];
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        if (q < narrow) nv[u][q] = wide_m ? Y[kk * N + q] : G[kk * M + q];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool value_row = (k + u * S) % R == 0;
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        if (q < narrow) {
                            acc[q] = fmaf(wv[u], nv[u][q], acc[q]);
                            if (value_row) bias[q] += wide_m ? (q == 0 ? wv[u] : 0.0f) : nv[u][q];
                        }
                }
            }
            for (; k < kend; k += S) {
                const size_t kk = size_t(k);
                const float wvv = wide_m ? G[kk * M + wi] : Y[kk * N + wi];
                const bool value_row = k % R == 0;
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    if (q < narrow) {
                        const float nvv = wide_m ? Y[kk * N + q] : G[kk * M + q];
                        acc[q] = fmaf(wvv, nvv, acc[q]);
                        if (value_row) bias[q] += wide_m ? (q == 0 ? wvv : 0.0f) : nvv;
                    }
            }
        }
        // wide_m: entries (wi, q) for q < N and the bias of row wi (in bias[0]);
        // otherwise entries (q, wi) for q < M, and bias[q] (the same in every
        // lane of a stream) is the bias of row q
        __syncthreads();  // readers of the previous wide chunk are done
#pragma unroll
        for (int q = 0; q < 16; ++q) red[threadIdx.x * 17 + q] = acc[q];
        red[threadIdx.x * 17 + 16] = wide_m ? bias[0] : 0.0f;
        __syncthreads();
        if (s == 0 && wi < wide) {
            float tot[17];
#pragma unroll
            for (int q = 0; q < 17; ++q) tot[q] = 0.0f;
            for (int ss = 0; ss < S; ++ss)
#pragma unroll
                for (int q = 0; q < 17; ++q) tot[q] += red[(ss * Wc + w) * 17 + q];
            if (wide_m) {
                for (int q = 0; q < N; ++q) P[size_t(wi) * (N + 1) + q] = tot[q];
                P[size_t(wi) * (N + 1) + N] = tot[16];
            } else {
                for (int q = 0; q < M; ++q) P[size_t(q) * (N + 1) + wi] = tot[q];
            }
        }
        if (!wide_m && w0 == 0) {
            __syncthreads();
            if (w == 0 && s < S)
#pragma unroll
                for (int q = 0; q < 16; ++q) red[s * 17 + q] = bias[q];
            __syncthreads();
            if (int(threadIdx.x) < M) {
                float b = 0.0f;
                for (int ss = 0; ss < S; ++ss) b += red[ss * 17 + threadIdx.x];
                P[size_t(threadIdx.x) * (N + 1) + N] = b;
            }
        }
    }
}

// Workgroups go to the eight XCDs round-robin (workgroup b on XCD b % 8), each
// XCD with its own L2.  This renumbering gives every XCD a contiguous range of
// work items, so that the tiles of one split, which read the same rows of G
// or Y, run under one L2.  It is a permutation of [0, n) for any n.
// The group whose range [begin[t], begin[t + 1]) holds b (b in [0,
// begin[count])).  Every boundary is loaded at once and compared, instead of a
// search whose every step waits on the load before it: kernel arguments come
// through the scalar cache, which is cold at each launch, so each such step
// costs a memory round trip before the workgroup's first real load.
__device__ __forceinline__ int group_of(const int (&begin)[kMaxTransitions + 1], int count, int b) {
    int t = 0;
#pragma unroll
    for (int k = 1; k < kMaxTransitions; ++k) t += (k < count && b >= begin[k]) ? 1 : 0;
    return t;
}

__device__ __forceinline__ int xcd_grouped(int b, int n) {
    const int x = b & 7, q = b >> 3, per = (n + 7) >> 3, full = (n & 7) ? (n & 7) : 8;
    return x < full ? x * per + q : full * per + (x - full) * (per - 1) + q;
}

// Two workgroups per CU (LDS 2 x 67.6 KB): one's chunk loads and barriers
// overlap the other's MFMAs.
__global__ __launch_bounds__(256, 2) void wgrad_grouped_kernel(WgradArgs a) {
    __shared__ __attribute__((aligned(16))) float lds[kWgLds];
    static_assert(256 * 17 <= kWgLds, "thin-transition scratch exceeds the shared LDS");
    const int b = xcd_grouped(int(blockIdx.x), int(gridDim.x));
    const int t = group_of(a.block_begin, a.transitions, b);
    const int local = b - a.block_begin[t];
    if (a.M[t] <= 16 || a.N[t] <= 16) wgrad_thin(a, t, local, lds);
    else if (a.tile[t] == 64) wgrad_tile<64>(a, t, local, lds);
    else wgrad_tile<128>(a, t, local, lds);
}

// Optimizers: one launch covers every transition.  Each transition's buffers
// are separate allocations; the launch carries their pointers by value.
constexpr int kOptimizerThreads = 256;

// Chunks of an update launch's own finiteness test (OptimizerArgs::test),
// kOptimizerThreads entries each: every lane loads its entry of every one, so
// their number is kept small (10,240 entries and fewer, about).
constexpr int kTestChunks = 40;

struct OptimizerArgs {
    float* W[kMaxTransitions];
    float* S[kMaxTransitions];   // RPROP step / Adam first moment
    float* Ga[kMaxTransitions];  // active gradient
    float* Gi[kMaxTransitions];  // inactive gradient / Adam second moment
    float* WT[kMaxTransitions];  // row-major copy of the weights, kept current by RPROP and Adam
    int NO[kMaxTransitions], NI[kMaxTransitions];
    int begin[kMaxTransitions + 1];
    int block_begin[kMaxTransitions + 1];  // blocks of kOptimizerThreads entries, per transition
    int transitions;
    // guarded: update only if the epoch's scalars pass the acceptance rule;
    // the first lane of the grid leaves the verdict in *verdict (if non-null)
    UpdateGuard guard;
    int guarded;
    int* verdict;
    // publish_dst non-null: the first workgroup copies publish_words 32-bit
    // words of the scalar block to its pinned host mirror (the download the
    // guarded update goes out behind), whether or not the update applies
    const unsigned* publish_src;
    unsigned* publish_dst;
    int publish_words;
    // test: the launch tests the active gradients for finiteness itself where
    // the rule would read the gradient totals (the transitions' entries make at
    // most kTestChunks chunks), and its first workgroup writes stats[t] = {0,
    // 0, whether transition t has a non-finite entry, none}, into the totals
    // and straight into the host mirror
    int test;
    GradStats* stats;
};

// The scalar block to the host, by the first workgroup of an update launch.
// A launch with its own finiteness test copies all but the gradient totals:
// test_gradients writes those.  No fence: the host block is coherent pinned
// memory, which the stores reach over the bus without passing a GPU cache,
// and the host reads it only after the launch's completion event (hipEvent-
// Synchronize), which orders the launch's writes before it.  (A system-scope
// fence here writes back the L2 first: 10.1 -> 9.2 us for the Poisson graph
// epoch's update launch without it.)
__device__ __forceinline__ void publish_scalars(const OptimizerArgs& a) {
    if (!a.publish_dst || blockIdx.x != 0) return;
    int skip_begin = 0, skip_end = 0;
    if (a.test) {
        skip_begin = int(reinterpret_cast<const unsigned*>(a.stats) - a.publish_src);
        skip_end = skip_begin + a.transitions * int(sizeof(GradStats) / sizeof(unsigned));
    }
    for (int i = threadIdx.x; i < a.publish_words; i += kOptimizerThreads)
        if (i < skip_begin || i >= skip_end) a.publish_dst[i] = a.publish_src[i];
}

// The launch's own finiteness test (OptimizerArgs::test): lane c lays chunk c
// of the transitions' entries out in LDS (where it starts, how many entries,
// which transition), then every lane loads its entry of every chunk at once
// (one round of loads for the whole network; a slot past the last chunk loads
// that chunk again, with no branch to hold the loads back), the workgroup ORs
// the transitions with a non-finite entry into one mask, and the first
// workgroup writes the totals.  Whether every entry is finite, on every lane.
__device__ bool test_gradients(const OptimizerArgs& a) {
    // chunk c: {address low and high words, its last entry's lane, transition}
    __shared__ int4 chunk[kTestChunks];
    __shared__ unsigned bad_mask;
    const int lane = threadIdx.x;
    int chunks = 0;
    for (int t = 0; t < a.transitions; ++t) {
        const int count = a.begin[t + 1] - a.begin[t];
        const int n = (count + kOptimizerThreads - 1) / kOptimizerThreads;
        if (lane >= chunks && lane < chunks + n && lane < kTestChunks) {
            const int start = (lane - chunks) * kOptimizerThreads;
            const unsigned long long p = reinterpret_cast<unsigned long long>(a.Ga[t] + start);
            chunk[lane] = make_int4(int(unsigned(p)), int(unsigned(p >> 32)),
                                    min(kOptimizerThreads, count - start) - 1, t);
        }
        chunks += n;
    }
    chunks = min(chunks, kTestChunks);
    if (lane == 0) bad_mask = 0;
    __syncthreads();
    // global (not flat) loads: a flat load would count against the LDS reads'
    // wait too
    typedef const __attribute__((address_space(1))) float* global_floats;
    int4 e[kTestChunks];
#pragma unroll
    for (int c = 0; c < kTestChunks; ++c) e[c] = chunk[min(c, chunks - 1)];
    float v[kTestChunks];
#pragma unroll
    for (int c = 0; c < kTestChunks; ++c) {
        const unsigned long long p = unsigned(e[c].x) | (static_cast<unsigned long long>(unsigned(e[c].y)) << 32);
        v[c] = reinterpret_cast<global_floats>(p)[min(lane, e[c].z)];
    }
    unsigned mask = 0;
#pragma unroll
    for (int c = 0; c < kTestChunks; ++c)
        if (!isfinite(v[c])) mask |= 1u << e[c].w;
    __syncthreads();  // bad_mask is cleared
    if (mask) atomicOr(&bad_mask, mask);
    __syncthreads();
    const unsigned m = bad_mask;
    if (blockIdx.x == 0 && a.publish_dst) {
        if (threadIdx.x < a.transitions) {
            const GradStats r{0.0, 0.0, (m >> threadIdx.x) & 1u, INT_MAX, 0};
            a.stats[threadIdx.x] = r;
            const int offset = int(reinterpret_cast<const unsigned*>(a.stats) - a.publish_src);
            reinterpret_cast<GradStats*>(a.publish_dst + offset)[threadIdx.x] = r;
        }
    } else if (blockIdx.x == 0 && threadIdx.x < a.transitions) {
        a.stats[threadIdx.x] = GradStats{0.0, 0.0, (m >> threadIdx.x) & 1u, INT_MAX, 0};
    }
    return m == 0;
}

// The guarded update's rule, the same on every lane of the grid; the first
// lane records it for the reductions that wait on it (ReduceArgs::gate).
// `finite`: the launch's own test of the gradients (OptimizerArgs::test_*).
__device__ __forceinline__ bool update_applies(const OptimizerArgs& a, bool finite = true) {
    if (!a.guarded) return true;
    const bool ok = finite && update_accepted(a.guard);
    if (a.verdict && blockIdx.x == 0 && threadIdx.x == 0) *a.verdict = ok ? 1 : 0;
    return ok;
}


// Entry j = o + NO*i of a weight block into its row-major copy (bias column i = NI excluded).
__device__ __forceinline__ void copy_transposed(const OptimizerArgs& a, int t, int j, float w) {
    const int i = j / a.NO[t], o = j - i * a.NO[t];
    if (i < a.NI[t]) a.WT[t][i + a.NI[t] * o] = w;
}


// The entry's optimizer state, loaded apart from the update so that a caller
// can send the loads out before its gradient is complete.
struct RpropState {
    float w, step, gi;
};
__device__ __forceinline__ RpropState rprop_state(const OptimizerArgs& a, int t, int j) {
    return RpropState{a.W[t][j], a.S[t][j], a.Gi[t][j]};
}

// Resile_k (cuda/derivative_kernels_v4.cu:752-778) on entry j of transition t
// with gradient g and state e: sign tests on float products, the gradient kept
// (or zeroed on a rollback or a rejected step) in the active buffer.  The
// optimizers round every product and sum separately, as the reference's CPU
// build does: no multiply-add contraction (hipcc contracts by default, and
// __fmul_rn/__fadd_rn do not prevent it).
__device__ __forceinline__ void rprop_update(const OptimizerArgs& a, int t, int j, float g, const RpropState& e) {
#pragma clang fp contract(off)
    const float gi = e.gi;
    const float prod = g * gi;
    float s = e.step;
    if (prod > 0) s *= 1.2f;
    const float w = e.w;
    const float nW = w - copysignf(s, g);
    float kept = w, kept_g = g;
    if (prod < 0) {
        kept = w + copysignf(s, gi);
        s *= 0.5f;
        kept_g = 0.0f;
    } else if (g != 0.0f) {
        if (fabsf(nW) <= 20.0f) kept = nW;
        else {
            s = 0.1f;
            kept_g = 0.0f;
        }
    }
    a.Ga[t][j] = kept_g;
    a.W[t][j] = kept;
    a.S[t][j] = s;
    copy_transposed(a, t, j, kept);
}

// grad_t[m + M*n] (+)= sum over splits of the partials of entry (m, n), n = N
// being the bias.  Split-major partials ([split][entry]): block = 64 consecutive
// entries x 4 waves, wave w sums splits w + 4u (+ 64i) into running sum u
// (sixteen, combined in a fixed tree), then the four wave sums in wave order.
// Split-minor partials ([entry][split]): one wave per entry, lane l sums splits
// l + 64u (+ 1024i) into running sum u (sixteen, combined in a fixed tree),
// then a fixed shuffle tree.  Either way the summation order is fixed whatever
// the scheduling.
__device__ void finish_costs(const ReduceArgs& a);
template <int THREADS>
__device__ void graph_stage(const GraphLaunch& g);
template <int THREADS>
__device__ void graph_run(const GraphLaunch& g, bool fresh);

// UPDATE: the lane that finishes an entry's gradient applies RPROP to it
// (reduce_rprop_kernel), which is the reduction followed by rprop_kernel in one
// launch, bit for bit; it loads the entry's optimizer state (and, accumulating,
// its gradient) before the partials, so that the two loads' latencies overlap.
// Block 0 finishes the costs and evaluates the graph when the launch carries
// them: the longest chain of the launch is dispatched first, and the graph's
// nodes are loaded before the costs are finished.
template <bool UPDATE>
__device__ __forceinline__ void reduce_grouped(const ReduceArgs& a, const OptimizerArgs& o) {
    __shared__ float part[2][4][64];
    const int cost_block = a.costs || a.with_graph ? 1 : 0;
    if (cost_block && blockIdx.x == 0) {
        if (a.with_graph) graph_stage<256>(a.graph);
        finish_costs(a);
        if (a.with_graph) graph_run<256>(a.graph, true);
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int block = int(blockIdx.x) - cost_block;
    const int t = group_of(a.block_begin, a.transitions, block);
    const int local = block - a.block_begin[t];
    const int M = a.M[t], N1 = a.N[t] + 1, S = a.splits[t];
    const int count = M * N1;
    // where entry j of transition t lives in the gradient and optimizer buffers
    auto index_of = [&](int j) {
        const int mrow = j / N1, n = j - mrow * N1;
        return mrow + M * n;
    };
    // Sixteen running sums per lane, each fed by an unconditional load (an
    // index past the last split reads the last split and adds nothing), so a
    // round's sixteen loads are in flight together; the sums then meet in a
    // fixed tree.
    constexpr int U = 16;
    auto tree = [](float (&acc)[U]) {
#pragma unroll
        for (int w = 1; w < U; w *= 2)
#pragma unroll
            for (int u = 0; u < U; u += 2 * w) acc[u] += acc[u + w];
        return acc[0];
    };
    // A second pass's partials (splits2 > 0) are summed in the same rounds of
    // loads as the first's, each into running sums of its own, so the two
    // sums are what two rounds in turn give, bit for bit.
    const bool two = a.splits2[t] > 0;  // uniform over the block
    const int S2 = two ? a.splits2[t] : 0, Smax = max(S, S2);
    if (!a.split_minor[t]) {
        const size_t stride = size_t(count);
        const int j = local * 64 + lane;
        const bool finisher = wave == 0 && j < count;
        const int idx = finisher ? index_of(j) : 0;
        RpropState e{};
        float before = 0.0f;
        if (finisher) {
            if constexpr (UPDATE) e = rprop_state(o, t, idx);
            if (a.accumulate) before = a.grad[t][idx];
        }
        // every wave; the sums of entry j are valid on wave 0's lane
        float s1 = 0.0f, s2 = 0.0f;
        if (j < count) {
            const float* P1 = a.partial[t] + j;
            const float* P2 = two ? a.partial2[t] + j : P1;
            float acc1[U], acc2[U];
#pragma unroll
            for (int u = 0; u < U; ++u) acc1[u] = acc2[u] = 0.0f;
            for (int q = wave; q < Smax; q += 4 * U) {  // wave w: splits w, w + 4, ...
                float v1[U], v2[U];
#pragma unroll
                for (int u = 0; u < U; ++u) v1[u] = P1[size_t(min(q + 4 * u, S - 1)) * stride];
                if (two)
#pragma unroll
                    for (int u = 0; u < U; ++u) v2[u] = P2[size_t(min(q + 4 * u, S2 - 1)) * stride];
#pragma unroll
                for (int u = 0; u < U; ++u) acc1[u] += q + 4 * u < S ? v1[u] : 0.0f;
                if (two)
#pragma unroll
                    for (int u = 0; u < U; ++u) acc2[u] += q + 4 * u < S2 ? v2[u] : 0.0f;
            }
            s1 = tree(acc1);
            if (two) s2 = tree(acc2);
        }
        part[0][wave][lane] = s1;
        part[1][wave][lane] = s2;
        __syncthreads();
        const float sum = (part[0][0][lane] + part[0][1][lane]) + (part[0][2][lane] + part[0][3][lane]);
        const float sum2 = (part[1][0][lane] + part[1][1][lane]) + (part[1][2][lane] + part[1][3][lane]);
        if (finisher) {
            float v = a.accumulate ? before + sum : sum;
            if (two) v = v + sum2;
            if constexpr (UPDATE) rprop_update(o, t, idx, v, e);
            else if (!a.gate || *a.gate) a.grad[t][idx] = v;
        }
    } else {
        const int j = local * 4 + wave;
        if (j >= count) return;
        const int idx = index_of(j);
        RpropState e{};
        float before = 0.0f;
        if (lane == 0) {
            if constexpr (UPDATE) e = rprop_state(o, t, idx);
            if (a.accumulate) before = a.grad[t][idx];
        }
        // the sums of entry j, valid on lane 0
        const float* P1 = a.partial[t] + size_t(j) * S;
        const float* P2 = two ? a.partial2[t] + size_t(j) * S2 : P1;
        float acc1[U], acc2[U];
#pragma unroll
        for (int u = 0; u < U; ++u) acc1[u] = acc2[u] = 0.0f;
        for (int q = lane; q < Smax + 63; q += 64 * U) {  // lane l: splits l, l + 64, ...
            float v1[U], v2[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v1[u] = P1[min(q + 64 * u, S - 1)];
            if (two)
#pragma unroll
                for (int u = 0; u < U; ++u) v2[u] = P2[min(q + 64 * u, S2 - 1)];
#pragma unroll
            for (int u = 0; u < U; ++u) acc1[u] += q + 64 * u < S ? v1[u] : 0.0f;
            if (two)
#pragma unroll
                for (int u = 0; u < U; ++u) acc2[u] += q + 64 * u < S2 ? v2[u] : 0.0f;
        }
        float s = tree(acc1), s2 = 0.0f;
        for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off, 64);
        if (two) {
            s2 = tree(acc2);
            for (int off = 32; off > 0; off >>= 1) s2 += __shfl_down(s2, off, 64);
        }
        if (lane == 0) {
            float v = a.accumulate ? before + s : s;
            if (two) v = v + s2;
            if constexpr (UPDATE) rprop_update(o, t, idx, v, e);
            else if (!a.gate || *a.gate) a.grad[t][idx] = v;
        }
    }
}

__global__ __launch_bounds__(256) void reduce_grouped_kernel(ReduceArgs a) { reduce_grouped<false>(a, OptimizerArgs{}); }

__global__ __launch_bounds__(256) void reduce_rprop_kernel(ReduceArgs a, OptimizerArgs o) {
    reduce_grouped<true>(a, o);
}
// Direct weight-gradient tiles, for short reductions: a workgroup owns one
// 64x64 tile of dW over its split's columns, and its four waves take the
// split's 4-column groups in turn (wave w: groups w, w + 4, ...).  Operands
// come straight from global memory into registers, no LDS staging: lane l
// loads the float4 G[c][m0 + 4(l%16) .. +3] and Y[c][n0 + 4(l%16) .. +3] of
// column c = c0 + l/16, and that pair feeds sixteen v_mfma_f32_16x16x4f32 --
// tile (tr, tc) takes component tr of the G float4 as A[l%16][l/16] and
// component tc of the Y float4 as B[l/16][l%16], so its accumulator register
// v of lane l is dW(m0 + 4(4(l/16) + v) + tr, n0 + 4(l%16) + tc).  The
// workgroup then sums its four waves' tiles in LDS in the fixed order
// (w0 + w2) + (w1 + w3) and writes its split's partial, as the LDS-staged
// tiles do.  The bias (n-tile 0 only) is the sum of G over value-row columns.
constexpr int kWdSlot = 64 * 64;                // one 64x64 tile in LDS, float4 per (x, z, lane)
constexpr int kWdLds = 2 * kWdSlot + 256;       // two tiles; also the thin roles' 256 x 17 scratch
constexpr int kWdBiasAhead = 4;                 // bias column groups loaded before the tile's epilogue
#ifndef CPDE_WD_DEPTH
#define CPDE_WD_DEPTH 2
#endif
constexpr int kWdDepth = CPDE_WD_DEPTH;        // column groups loaded ahead

// 4 consecutive entries [w0, w0 + 4) of row c of a [column][width] stack
// (offset = c * width + w0).  MASK: zeros beyond the width -- VEC (width % 4
// == 0) then loads the float4 only where it is inside; unmasked, the load is
// unconditional (full tiles).
template <bool VEC, bool MASK>
__device__ __forceinline__ float4 wd_load(const float* __restrict__ base, unsigned offset, int w0, int width) {
    const float* p = base + offset;
    if constexpr (!MASK) {
        return *reinterpret_cast<const float4*>(p);
    } else if constexpr (VEC) {
        return w0 < width ? *reinterpret_cast<const float4*>(p) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (w0 + 0 < width) v.x = p[0];
        if (w0 + 1 < width) v.y = p[1];
        if (w0 + 2 < width) v.z = p[2];
        if (w0 + 3 < width) v.w = p[3];
        return v;
    }
}

// The main loop of a direct tile: acc += this wave's columns of G^T Y.
template <bool VEC, bool MASK>
__device__ __forceinline__ void wd_accumulate(floatx4 (&acc)[4][4], const float* __restrict__ G,
                                              const float* __restrict__ Y, int M, int N, int kbegin, int kend,
                                              int gm, int yn, int wave, int q) {
    auto mma = [&](const float4 g, const float4 y) {
        const float gv[4] = {g.x, g.y, g.z, g.w}, yv[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int z = 0; z < 4; ++z)
                acc[x][z] = __builtin_amdgcn_mfma_f32_16x16x4f32(gv[x], yv[z], acc[x][z], 0, 0, 0);
    };
    // full steps of 16 columns (this wave's column c = kbegin + 16 s + 4 wave + q),
    // loaded kWdDepth steps ahead; then at most one partial step with the
    // columns beyond the split zeroed.  The steady-state loop is branch-free,
    // so the loads stay in flight across its iterations.
    const int full = (kend - kbegin) / 16;
    const unsigned c0 = unsigned(kbegin + 4 * wave + q);
    unsigned go = c0 * unsigned(M) + unsigned(gm), yo = c0 * unsigned(N) + unsigned(yn);
    const unsigned gstep = 16u * unsigned(M), ystep = 16u * unsigned(N);
    if (full >= kWdDepth) {
        float4 gb[kWdDepth], yb[kWdDepth];
#pragma unroll
        for (int d = 0; d < kWdDepth; ++d) {
            gb[d] = wd_load<VEC, MASK>(G, go, gm, M);
            yb[d] = wd_load<VEC, MASK>(Y, yo, yn, N);
            go += gstep;
            yo += ystep;
        }
        int s0 = 0;
        // two register sets in turn (no copies between them): each half of
        // the body sends the other set's next kWdDepth steps of loads out
        // before its own products, so a set's loads stay in flight across the
        // other set's products
        float4 gn[kWdDepth], yn4[kWdDepth];
        auto fetch = [&](float4 (&gs)[kWdDepth], float4 (&ys)[kWdDepth]) {
#pragma unroll
            for (int d = 0; d < kWdDepth; ++d) {
                gs[d] = wd_load<VEC, MASK>(G, go, gm, M);
                ys[d] = wd_load<VEC, MASK>(Y, yo, yn, N);
                go += gstep;
                yo += ystep;
            }
        };
        auto products = [&](const float4 (&gs)[kWdDepth], const float4 (&ys)[kWdDepth]) {
#pragma unroll
            for (int d = 0; d < kWdDepth; ++d) mma(gs[d], ys[d]);
        };
#pragma unroll 1
        for (; s0 + 3 * kWdDepth <= full; s0 += 2 * kWdDepth) {
            fetch(gn, yn4);
            __builtin_amdgcn_sched_barrier(0);
            products(gb, yb);
            fetch(gb, yb);
            __builtin_amdgcn_sched_barrier(0);
            products(gn, yn4);
        }
        if (s0 + 2 * kWdDepth <= full) {  // one more set of steps fits before the tail
            fetch(gn, yn4);
            __builtin_amdgcn_sched_barrier(0);
            products(gb, yb);
#pragma unroll
            for (int d = 0; d < kWdDepth; ++d) {
                gb[d] = gn[d];
                yb[d] = yn4[d];
            }
            s0 += kWdDepth;
        }
        // steps s0 .. s0 + kWdDepth - 1 are loaded; fewer than kWdDepth full steps follow
#pragma unroll
        for (int d = 0; d < kWdDepth; ++d) mma(gb[d], yb[d]);
        for (int s = s0 + kWdDepth; s < full; ++s) {
            mma(wd_load<VEC, MASK>(G, go, gm, M), wd_load<VEC, MASK>(Y, yo, yn, N));
            go += gstep;
            yo += ystep;
        }
    } else {
        for (int s = 0; s < full; ++s) {
            mma(wd_load<VEC, MASK>(G, go, gm, M), wd_load<VEC, MASK>(Y, yo, yn, N));
            go += gstep;
            yo += ystep;
        }
    }
    if (full * 16 < kend - kbegin) {
        const int c = kbegin + 16 * full + 4 * wave + q;
        float4 g = make_float4(0.0f, 0.0f, 0.0f, 0.0f), y = g;
        if (c < kend) {
            g = wd_load<VEC, MASK>(G, unsigned(c) * unsigned(M) + unsigned(gm), gm, M);
            y = wd_load<VEC, MASK>(Y, unsigned(c) * unsigned(N) + unsigned(yn), yn, N);
        }
        mma(g, y);
    }
}

template <bool VEC>
__device__ __forceinline__ void wgrad_direct_tile(const WgradArgs& a, int t, int local, float* lds) {
    const int M = a.M[t], N = a.N[t], K = a.K[t], R = a.R[t];
    const int tiles_m = (M + 63) / 64, tiles_n = (N + 63) / 64;
    const int tile = local % (tiles_m * tiles_n), split = local / (tiles_m * tiles_n);
    const int m0 = (tile % tiles_m) * 64, n0 = (tile / tiles_m) * 64;
    const int kbegin = split * a.kchunk[t], kend = min(K, kbegin + a.kchunk[t]);
    const float* __restrict__ G = a.G[t];
    const float* __restrict__ Y = a.Y[t];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
    const int gm = m0 + 4 * j, yn = n0 + 4 * j;
    floatx4 acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    if (VEC && m0 + 64 <= M && n0 + 64 <= N) wd_accumulate<VEC, false>(acc, G, Y, M, N, kbegin, kend, gm, yn, wave, q);
    else wd_accumulate<VEC, true>(acc, G, Y, M, N, kbegin, kend, gm, yn, wave, q);
    // bias (n-tile 0): the sum of G over the split's value-row columns; lane
    // group (wave, q) takes value columns first + R (4 wave + q + 16 i) for its
    // 4 rows, the sixteen groups then meet in a fixed order.  The first
    // kWdBiasAhead columns of each group are loaded now (an index past the
    // split reads its last column and is not added), so that their latency
    // passes under the tile's epilogue, whose barriers wait on LDS only.
    const bool with_bias = n0 == 0;
    const int bias_c0 = (kbegin + R - 1) / R * R + R * (4 * wave + q);
    float4 bias_ahead[kWdBiasAhead];
    if (with_bias)
#pragma unroll
        for (int u = 0; u < kWdBiasAhead; ++u) {
            const int c = min(bias_c0 + 16 * R * u, kend - 1);
            bias_ahead[u] = wd_load<VEC, true>(G, unsigned(c) * unsigned(M) + unsigned(gm), gm, M);
        }
    // (w0 + w2) + (w1 + w3): waves 2 and 3 put their tiles in the two LDS
    // slots, waves 0 and 1 add them and put w0 + w2 and w1 + w3 back, each
    // lane's accumulator quad (x, z) as one float4 at ((4x + z) 64 + lane) 4;
    // then every lane adds the two sums of 16 entries, a wave writing one
    // 64-entry row of the partial per instruction
    auto slot = [&](int k, int x, int z) {
        return reinterpret_cast<floatx4*>(lds + k * kWdSlot + ((4 * x + z) * 64 + lane) * 4);
    };
    if (wave >= 2)
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int z = 0; z < 4; ++z) *slot(wave - 2, x, z) = acc[x][z];
    __syncthreads();
    if (wave < 2)
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int z = 0; z < 4; ++z) {
                floatx4* p = slot(wave, x, z);
                *p = acc[x][z] + *p;
            }
    __syncthreads();
    float* P = a.partial[t] + size_t(split) * M * (N + 1);
    if (n0 + lane < N) {
        // entry (row ml, column lane) of the tile: accumulator quad
        // (x, z) = (ml % 4, lane % 4) of lane 16 (ml / 16) + lane / 4, component (ml / 4) % 4
        const int zl = lane & 3, jl = lane >> 2;
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
            const int ml = wave + 4 * i;
            const int at = ((4 * (ml & 3) + zl) * 64 + 16 * (ml >> 4) + jl) * 4 + ((ml >> 2) & 3);
            if (m0 + ml < M) P[size_t(m0 + ml) * (N + 1) + n0 + lane] = lds[at] + lds[kWdSlot + at];
        }
    }
    if (with_bias) {
        float4 bias = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int u = 0; u < kWdBiasAhead; ++u)
            if (bias_c0 + 16 * R * u < kend) {
                bias.x += bias_ahead[u].x;
                bias.y += bias_ahead[u].y;
                bias.z += bias_ahead[u].z;
                bias.w += bias_ahead[u].w;
            }
        for (int c = bias_c0 + 16 * R * kWdBiasAhead; c < kend; c += 16 * R) {
            const float4 g = wd_load<VEC, true>(G, unsigned(c) * unsigned(M) + unsigned(gm), gm, M);
            bias.x += g.x;
            bias.y += g.y;
            bias.z += g.z;
            bias.w += g.w;
        }
        bias.x += __shfl_xor(bias.x, 16);
        bias.y += __shfl_xor(bias.y, 16);
        bias.z += __shfl_xor(bias.z, 16);
        bias.w += __shfl_xor(bias.w, 16);
        bias.x += __shfl_xor(bias.x, 32);
        bias.y += __shfl_xor(bias.y, 32);
        bias.z += __shfl_xor(bias.z, 32);
        bias.w += __shfl_xor(bias.w, 32);
        float* bias_lds = lds + 2 * kWdSlot;  // past the two tile slots
        if (q == 0) {
            bias_lds[wave * 64 + 4 * j + 0] = bias.x;
            bias_lds[wave * 64 + 4 * j + 1] = bias.y;
            bias_lds[wave * 64 + 4 * j + 2] = bias.z;
            bias_lds[wave * 64 + 4 * j + 3] = bias.w;
        }
        __syncthreads();
        if (wave == 0 && m0 + lane < M)
            P[size_t(m0 + lane) * (N + 1) + N] =
                (bias_lds[lane] + bias_lds[128 + lane]) + (bias_lds[64 + lane] + bias_lds[192 + lane]);
    }
}

// Direct tiles and the thin transitions' roles in one launch (33 KB of LDS
// per workgroup).
#ifndef CPDE_WD_MIN_BLOCKS
#define CPDE_WD_MIN_BLOCKS 3
#endif
__global__ __launch_bounds__(256, CPDE_WD_MIN_BLOCKS) void wgrad_direct_kernel(WgradArgs a) {
    __shared__ __attribute__((aligned(16))) float lds[kWdLds];
    static_assert(256 * 17 <= kWdLds, "thin-transition scratch exceeds the shared LDS");
    const int b = xcd_grouped(int(blockIdx.x), int(gridDim.x));
    const int t = group_of(a.block_begin, a.transitions, b);
    const int local = b - a.block_begin[t];
    if (a.M[t] <= 16 || a.N[t] <= 16) wgrad_thin(a, t, local, lds);
    else if (a.M[t] % 4 == 0 && a.N[t] % 4 == 0) wgrad_direct_tile<true>(a, t, local, lds);
    else wgrad_direct_tile<false>(a, t, local, lds);
}

void launch_wgrad_grouped(Device& d, const WgradArgs& a, double flops) {
    TraceScope trace(d, kTraceWgrad, flops);
    if (a.direct) hipLaunchKernelGGL(wgrad_direct_kernel, a.block_begin[a.transitions], 256, 0, d.stream, a);
    else hipLaunchKernelGGL(wgrad_grouped_kernel, a.block_begin[a.transitions], 256, 0, d.stream, a);
    HIP_CHECK(hipGetLastError());
}

// Algorithmic bytes of a reduction launch (partials read, gradient read and
// written, `extra` more floats per entry), and its grid: one more block when
// it finishes costs or evaluates the graph.
static double reduce_bytes(const ReduceArgs& a, int extra) {
    double bytes = 0;
    for (int t = 0; t < a.transitions; ++t)
        bytes += 4.0 * (a.begin[t + 1] - a.begin[t]) * (a.splits[t] + a.splits2[t] + (a.accumulate ? 2 : 1) + extra);
    for (int c = 0; c < a.costs; ++c) bytes += double(sizeof(CostStats)) * (a.cost_count[c] + 2);
    return bytes;
}
static unsigned reduce_grid(const ReduceArgs& a) {
    return unsigned(a.block_begin[a.transitions] + (a.costs || a.with_graph ? 1 : 0));
}

// The reduction of a gradient group followed by RPROP on the same
// transitions: transitions [first, first + a.transitions) of `net`, whose
// active gradient buffers are a.grad.
void launch_reduce_rprop(Device& d, const ReduceArgs& a, Net& net, int first) {
    OptimizerArgs o{};
    o.transitions = a.transitions;
    for (int k = 0; k < a.transitions; ++k) {
        const int t = first + k;
        const int act = net.active[t], inact = act == 1 ? 2 : 1;
        require(a.grad[k] == net.state[act][t], "fused update: gradient group is not the active buffer");
        o.W[k] = net.state[0][t];
        o.S[k] = net.state[3][t];
        o.Ga[k] = net.state[act][t];
        o.Gi[k] = net.state[inact][t];
        o.WT[k] = net.wt[t];
        o.NO[k] = net.neurons[t + 1];
        o.NI[k] = net.neurons[t];
    }
    TraceScope trace(d, kTraceSplitReduce, reduce_bytes(a, 6));
    hipLaunchKernelGGL(reduce_rprop_kernel, reduce_grid(a), 256, 0, d.stream, a, o);
    HIP_CHECK(hipGetLastError());
}

// Whether reduction `a` writes the gradient buffers of the network whose
// update is issued and not yet resolved (cpde_update_issue).
static bool into_issued_update(const Device& d, const ReduceArgs& a) {
    if (!d.issued.open || !d.issued.net) return false;
    const Net& n = *d.issued.net;
    for (int k = 0; k < a.transitions; ++k)
        for (size_t t = 0; t < n.state[1].size(); ++t)
            if (a.grad[k] == n.state[1][t] || a.grad[k] == n.state[2][t]) return true;
    return false;
}

// A reduction launched while an update is issued (the next epoch's first
// half, sent before this epoch's scalars are back) into that network's
// gradient stores only if the update applied: a rejected epoch leaves every
// state buffer as whole epochs leave it.
void launch_reduce_grouped(Device& d, const ReduceArgs& a) {
    TraceScope trace(d, kTraceSplitReduce, reduce_bytes(a, 0));
    ReduceArgs b = a;
    b.gate = into_issued_update(d, a) ? d.update_verdict : nullptr;
    hipLaunchKernelGGL(reduce_grouped_kernel, reduce_grid(b), 256, 0, d.stream, b);
    HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------------------------------
// Activation of a chunk (Server::activate, cuda/cpde_server.cu:158-170) and the
// evaluation copy-out (:180): wire layout [row][sample][channel] <-> stack.
// One lane per (point, row) of the chunk: copies that row's channels (32-bit
// index arithmetic; the host checks width * R fits).
__global__ void activate_kernel(float* __restrict__ x, const float* __restrict__ data, int data_width, int channels,
                                const int* __restrict__ rows, int R, int width, int offset, int valid) {
    const int total = width * R;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        const int p = e / R, r = e - p * R;
        float* dst = x + size_t(e) * channels;
        if (p < valid) {
            const float* src = data + (size_t(rows[r]) * data_width + offset + p) * channels;
            for (int c = 0; c < channels; ++c) dst[c] = src[c];
        } else {
            for (int c = 0; c < channels; ++c) dst[c] = 0.0f;
        }
    }
}

void launch_activate(Device& d, float* x, const float* data, int data_width, int channels, const int* rows_dev,
                     int rows, int width, int offset, int valid) {
    const size_t total = size_t(width) * rows;
    require(total < (size_t(1) << 31), "chunk too large for one activation");
    const int blocks = int(std::min<size_t>((total + 255) / 256, 4096));
    TraceScope trace(d, kTraceActivate, 8.0 * double(total) * channels);
    hipLaunchKernelGGL(activate_kernel, blocks, 256, 0, d.stream, x, data, data_width, channels, rows_dev, rows, width,
                       offset, valid);
    HIP_CHECK(hipGetLastError());
}

__global__ void output_kernel(float* __restrict__ dest, const float* __restrict__ out, int dest_width, int channels,
                              const int* __restrict__ rows, int R, int offset, int valid) {
    const int total = valid * R;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        const int p = e / R, r = e - p * R;
        const float* src = out + size_t(e) * channels;
        float* dst = dest + (size_t(rows[r]) * dest_width + offset + p) * channels;
        for (int c = 0; c < channels; ++c) dst[c] = src[c];
    }
}

void launch_output(Device& d, float* dest, const float* out, int dest_width, int channels, const int* rows_dev,
                   int rows, int width, int offset, int valid) {
    (void)width;
    const size_t total = size_t(valid) * rows;
    if (!total) return;
    require(total < (size_t(1) << 31), "chunk too large for one output copy");
    const int blocks = int(std::min<size_t>((total + 255) / 256, 4096));
    hipLaunchKernelGGL(output_kernel, blocks, 256, 0, d.stream, dest, out, dest_width, channels, rows_dev, rows, offset,
                       valid);
    HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------------------------------
// Deterministic reductions.  Cost statistics combine as a signed double sum plus
// the lexicographically smallest (sample, component) bad location
// (cuda/reduction_kernels.cuh:36-46); partials are reduced in a fixed order.
__device__ __forceinline__ CostStats combine(CostStats a, const CostStats& b) {
    a.value += b.value;
    if (b.bad_sample < a.bad_sample || (b.bad_sample == a.bad_sample && b.bad_component < a.bad_component)) {
        a.bad_sample = b.bad_sample;
        a.bad_component = b.bad_component;
    }
    return a;
}
__device__ __forceinline__ CostStats empty_cost() { return CostStats{0.0, INT_MAX, INT_MAX}; }
__device__ __forceinline__ void mark_bad(CostStats& s, int sample, int component) {
    s = combine(s, CostStats{0.0, sample, component});
}

// Block-wide fixed-order reduction: wave shuffles, then the 4 wave results in order.
__device__ CostStats block_reduce_cost(CostStats v) {
    __shared__ CostStats waves[kCostThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        CostStats o;
        o.value = __shfl_down(v.value, off, 64);
        o.bad_sample = __shfl_down(v.bad_sample, off, 64);
        o.bad_component = __shfl_down(v.bad_component, off, 64);
        v = combine(v, o);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) waves[wave] = v;
    __syncthreads();
    CostStats r = empty_cost();
    if (threadIdx.x == 0)
        for (int w = 0; w < kCostThreads / 64; ++w) r = combine(r, waves[w]);
    return r;
}

// One block of kCostThreads lanes: lane l combines records l, l + 256, ... in
// order (loaded four at a time, so that their latencies overlap: an index past
// the end reads the last record again and is not combined), then the fixed
// block reduction; the result overwrites or joins *total.
__device__ void finish_cost_records(const CostStats* __restrict__ records, int count, CostStats* __restrict__ total,
                                    int overwrite) {
    constexpr int U = 4;
    CostStats v = empty_cost();
    constexpr int step = kCostThreads;
    for (int i = threadIdx.x; i < count; i += U * step) {
        CostStats r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = records[min(i + u * step, count - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i + u * step < count) v = combine(v, r[u]);
    }
    v = block_reduce_cost(v);
    if (threadIdx.x == 0) *total = overwrite ? v : combine(*total, v);
}

// The cost finishes a reduction launch carries, on its cost block (256
// lanes): each cost's records combined exactly as finish_cost_records combines
// them (lane l: records l, l + 256, ... in order; then the fixed block
// reduction), so the same bits, but with every cost's records loaded in one
// go (four per lane and cost, an index past the end reading the last record
// again, not combined) and the trees side by side.  The finished totals stay
// in LDS for the graph (reduce_finished: the totals, their slots, how many).
__shared__ CostStats reduce_finished[kReduceCosts];
__shared__ const CostStats* reduce_finished_slot[kReduceCosts];
__shared__ int reduce_finished_count;

__device__ void finish_costs(const ReduceArgs& a) {
    constexpr int U = 4;
    __shared__ CostStats waves[kReduceCosts][kCostThreads / 64];
    constexpr int step = kCostThreads;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    CostStats v[kReduceCosts], prior[kReduceCosts];
    int rounds = 0;
#pragma unroll
    for (int c = 0; c < kReduceCosts; ++c) {
        v[c] = empty_cost();
        if (c < a.costs) {
            rounds = max(rounds, (a.cost_count[c] + U * step - 1) / (U * step));
            // a total joined rather than overwritten: loaded with the records
            if (threadIdx.x == 0 && !a.cost_overwrite[c]) prior[c] = *a.cost_total[c];
        }
    }
    for (int k = 0; k < rounds; ++k) {
        CostStats r[kReduceCosts][U];
#pragma unroll
        for (int c = 0; c < kReduceCosts; ++c)
            if (c < a.costs && a.cost_count[c] > 0) {
                const int count = a.cost_count[c];
#pragma unroll
                for (int u = 0; u < U; ++u)
                    r[c][u] = a.cost_partials[c][min(int(threadIdx.x) + (k * U + u) * step, count - 1)];
            }
#pragma unroll
        for (int c = 0; c < kReduceCosts; ++c)
            if (c < a.costs) {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (int(threadIdx.x) + (k * U + u) * step < a.cost_count[c]) v[c] = combine(v[c], r[c][u]);
            }
    }
#pragma unroll
    for (int c = 0; c < kReduceCosts; ++c)
        if (c < a.costs) {
            CostStats x = v[c];
            for (int off = 32; off > 0; off >>= 1) {
                CostStats o;
                o.value = __shfl_down(x.value, off, 64);
                o.bad_sample = __shfl_down(x.bad_sample, off, 64);
                o.bad_component = __shfl_down(x.bad_component, off, 64);
                x = combine(x, o);
            }
            if (lane == 0) waves[c][wave] = x;
        }
    __syncthreads();
    if (threadIdx.x == 0)
#pragma unroll
        for (int c = 0; c < kReduceCosts; ++c)
            if (c < a.costs) {
                CostStats r = empty_cost();
                for (int w = 0; w < step / 64; ++w) r = combine(r, waves[c][w]);
                const CostStats total = a.cost_overwrite[c] ? r : combine(prior[c], r);
                *a.cost_total[c] = total;
                reduce_finished[c] = total;
                reduce_finished_slot[c] = a.cost_total[c];
            }
    if (threadIdx.x == 0) reduce_finished_count = a.costs;
    __syncthreads();
}

__global__ __launch_bounds__(kCostThreads) void cost_finish_kernel(const CostStats* __restrict__ blocks, int count,
                                                                   CostStats* __restrict__ total, int overwrite) {
    finish_cost_records(blocks, count, total, overwrite);
}

static int cost_blocks_for(int count) { return std::max(1, std::min(kMaxCostBlocks, (count + kCostThreads - 1) / kCostThreads)); }

// First stage for long record lists: block b combines records [b*per, (b+1)*per)
// in order into out[b].
__global__ __launch_bounds__(kCostThreads) void cost_stage_kernel(const CostStats* __restrict__ in, int count, int per,
                                                                  CostStats* __restrict__ out) {
    CostStats v = empty_cost();
    const int begin = blockIdx.x * per, end = min(count, begin + per);
    for (int i = begin + threadIdx.x; i < end; i += blockDim.x) v = combine(v, in[i]);
    v = block_reduce_cost(v);
    if (threadIdx.x == 0) out[blockIdx.x] = v;
}

void launch_finish_cost(Device& d, const CostStats* partials, int blocks, int cost_index) {
    TraceScope trace(d, kTraceReduce, double(sizeof(CostStats)) * (blocks + 2));
    if (blocks > kMaxCostBlocks) {
        const int per = (blocks + kMaxCostBlocks - 1) / kMaxCostBlocks;
        const int staged = (blocks + per - 1) / per;
        hipLaunchKernelGGL(cost_stage_kernel, staged, kCostThreads, 0, d.stream, partials, blocks, per, d.cost_blocks);
        HIP_CHECK(hipGetLastError());
        partials = d.cost_blocks;
        blocks = staged;
    }
    hipLaunchKernelGGL(cost_finish_kernel, 1, kCostThreads, 0, d.stream, partials, blocks,
                       d.cost_totals + cost_index, int(d.take_fresh(cost_index)));
    HIP_CHECK(hipGetLastError());
}

static void finish_cost(Device& d, int blocks, int cost_index) { launch_finish_cost(d, d.cost_blocks, blocks, cost_index); }

__global__ void clear_costs_kernel(CostStats* c, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += blockDim.x * gridDim.x) c[i] = empty_cost();
}

// Workspace::begin (cuda/reduction_kernels.cuh:149-152) without a launch: the
// slots are marked fresh and the first finish into each overwrites it.
void launch_costs_begin(Device& d, int costs) {
    d.reserve_costs(costs);
    if (int(d.slot_fresh.size()) < costs) d.slot_fresh.resize(costs, 0);
    std::fill(d.slot_fresh.begin(), d.slot_fresh.begin() + costs, 1);
}

void launch_clear_fresh(Device& d, int count) {
    for (int i = 0; i < count && i < int(d.slot_fresh.size()); ++i)
        if (d.take_fresh(i)) {
            hipLaunchKernelGGL(clear_costs_kernel, 1, 64, 0, d.stream, d.cost_totals + i, 1);
            HIP_CHECK(hipGetLastError());
        }
}

// Array-matching squared loss (cuda/cost_kernels.cuh:6-35) on the output stack
// y [point][row][outputs]; g receives dE/dy.  One lane per (point, component):
// each lane forms w (y - t)^2 and 2 w (y - t); the per-point loss is then
// summed in fp32 in component order (as the reference does) by one lane per
// point, promoted to double, and reduced over the block in a fixed order.
// Blocks loop over groups of 256 / (rows*outputs) points.
__global__ __launch_bounds__(kCostThreads) void matching_kernel(
    const float* __restrict__ y, float* __restrict__ g, const float* __restrict__ target, int target_width,
    const int* __restrict__ target_rows, const float* __restrict__ weights, int weight_samples, int R, int outputs,
    int width, int valid, int offset, int collect, int gradient, CostStats* __restrict__ partials) {
    extern __shared__ float terms[];
    const int RO = R * outputs;
    const int ppb = max(1, kCostThreads / RO);
    CostStats local = empty_cost();
    for (int p0 = blockIdx.x * ppb; p0 < width; p0 += gridDim.x * ppb) {
        for (int e = threadIdx.x; e < ppb * RO; e += blockDim.x) {
            const int pl = e / RO, c = e - pl * RO;
            const int p = p0 + pl;
            float term = 0.0f;
            if (p < width) {
                const int d = c / outputs, o = c - d * outputs;
                const size_t i = size_t(p) * RO + c;
                float gi = 0.0f;
                if (p < valid) {
                    const int wp = weight_samples == 1 ? 0 : offset + p;
                    const float w = weights[(size_t(d) * weight_samples + wp) * outputs + o];
                    if (w != 0.0f) {
                        const float r = y[i] - target[(size_t(target_rows[d]) * target_width + offset + p) * outputs + o];
                        term = w * r * r;
                        gi = 2.0f * w * r;
                    }
                }
                if (gradient) {
                    g[i] = gi;
                    if (p < valid && !isfinite(gi)) mark_bad(local, offset + p, c);
                }
            }
            terms[e] = term;
        }
        __syncthreads();
        if (int(threadIdx.x) < ppb && p0 + int(threadIdx.x) < width) {
            const int p = p0 + threadIdx.x;
            float value = 0.0f;
            for (int c = 0; c < RO; ++c) value += terms[threadIdx.x * RO + c];
            if (!isfinite(value)) mark_bad(local, offset + p, -1);
            if (collect) local.value += double(value);
        }
        __syncthreads();
    }
    local = block_reduce_cost(local);
    if (threadIdx.x == 0) partials[blockIdx.x] = local;
}

void launch_matching(Device& d, const Plan& p, const float* y, float* g, const float* target, int target_width,
                     const int* target_rows, const float* weights, int weight_samples, int offset, int valid,
                     int cost_index, bool collect, bool gradient) {
    const int outputs = p.net->neurons.back();
    const int RO = p.rows * outputs;
    require(RO <= 16384, "matching cost: rows x outputs exceeds 16384");
    const int ppb = std::max(1, kCostThreads / RO);
    const int blocks = std::max(1, std::min(kMaxCostBlocks, (p.width + ppb - 1) / ppb));
    const size_t lds = sizeof(float) * size_t(ppb) * RO;
    {
    // y and target read, g written
    TraceScope trace(d, kTraceCost, 12.0 * double(p.columns()) * outputs);
    hipLaunchKernelGGL(matching_kernel, blocks, kCostThreads, lds, d.stream, y, g, target, target_width, target_rows,
                       weights, weight_samples, p.rows, outputs, p.width, valid, offset, int(collect), int(gradient),
                       d.cost_blocks);
    HIP_CHECK(hipGetLastError());
    }
    finish_cost(d, blocks, cost_index);
}

// Sparse linear/quadratic residuals (cuda/cost_kernels.cuh:37-90); component
// index = row*outputs + output.
__device__ __forceinline__ size_t component_at(int index, int outputs, int R, int p) {
    return (size_t(p) * R + index / outputs) * outputs + index % outputs;
}

__global__ __launch_bounds__(kCostThreads) void polynomial_kernel(
    const float* __restrict__ y, float* __restrict__ g, const cpde_poly_term* __restrict__ terms, int term_count,
    const float* __restrict__ coefficients, const float* __restrict__ rhs, const float* __restrict__ weights,
    int equations, int samples, int R, int outputs, int width, int valid, int offset, int collect, int gradient,
    CostStats* __restrict__ partials) {
    CostStats local = empty_cost();
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < width; p += blockDim.x * gridDim.x) {
        if (gradient)
            for (int k = 0; k < R * outputs; ++k) g[size_t(p) * R * outputs + k] = 0.0f;
        float total = 0.0f;
        if (p < valid)
            for (int e = 0; e < equations; ++e) {
                const int sample = offset + p;
                const float w = weights[size_t(e) * samples + sample];
                if (w == 0.0f) continue;
                float r = -rhs[size_t(e) * samples + sample];
                for (int t = 0; t < term_count; ++t) {
                    if (terms[t].equation != e) continue;
                    const float c = coefficients[size_t(t) * samples + sample];
                    if (c == 0.0f) continue;
                    const float a = y[component_at(terms[t].a, outputs, R, p)];
                    r += c * a * (terms[t].b < 0 ? 1.0f : y[component_at(terms[t].b, outputs, R, p)]);
                }
                total += w * r * r;
                const float scale = 2.0f * w * r;
                if (gradient)
                    for (int t = 0; t < term_count; ++t) {
                        if (terms[t].equation != e) continue;
                        const float c = coefficients[size_t(t) * samples + sample];
                        if (c == 0.0f) continue;
                        if (terms[t].b < 0) {
                            g[component_at(terms[t].a, outputs, R, p)] += scale * c;
                        } else {
                            g[component_at(terms[t].a, outputs, R, p)] +=
                                scale * c * y[component_at(terms[t].b, outputs, R, p)];
                            g[component_at(terms[t].b, outputs, R, p)] +=
                                scale * c * y[component_at(terms[t].a, outputs, R, p)];
                        }
                    }
            }
        if (!isfinite(total)) mark_bad(local, offset + p, -1);
        if (collect) local.value += double(total);
        if (gradient && p < valid)
            for (int k = 0; k < R * outputs; ++k)
                if (!isfinite(g[size_t(p) * R * outputs + k])) mark_bad(local, offset + p, k);
    }
    local = block_reduce_cost(local);
    if (threadIdx.x == 0) partials[blockIdx.x] = local;
}

void launch_polynomial(Device& d, const Plan& p, const float* y, float* g, const cpde_poly_term* terms, int term_count,
                       const float* coefficients, const float* rhs, const float* weights, int equations, int samples,
                       int offset, int valid, int cost_index, bool collect, bool gradient) {
    const int outputs = p.net->neurons.back();
    const int blocks = cost_blocks_for(p.width);
    hipLaunchKernelGGL(polynomial_kernel, blocks, kCostThreads, 0, d.stream, y, g, terms, term_count, coefficients, rhs,
                       weights, equations, samples, p.rows, outputs, p.width, valid, offset, int(collect),
                       int(gradient), d.cost_blocks);
    HIP_CHECK(hipGetLastError());
    finish_cost(d, blocks, cost_index);
}

// Per-sample expression densities -> cost slot (cost_graph::sample_blocks,
// cuda/cost_graph.cuh:35-43).  bad[p] == -2 means clean.
__global__ __launch_bounds__(kCostThreads) void sample_blocks_kernel(const double* __restrict__ values,
                                                                     const int* __restrict__ bad, int valid, int offset,
                                                                     CostStats* __restrict__ partials) {
    CostStats local = empty_cost();
    for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < valid; p += blockDim.x * gridDim.x) {
        local.value += values[p];
        if (bad[p] != -2) mark_bad(local, offset + p, bad[p]);
    }
    local = block_reduce_cost(local);
    if (threadIdx.x == 0) partials[blockIdx.x] = local;
}

void launch_sample_reduce(Device& d, const double* values, const int* bad, int valid, int offset, int cost_index) {
    const int blocks = cost_blocks_for(valid);
    hipLaunchKernelGGL(sample_blocks_kernel, blocks, kCostThreads, 0, d.stream, values, bad, valid, offset,
                       d.cost_blocks);
    HIP_CHECK(hipGetLastError());
    finish_cost(d, blocks, cost_index);
}

__global__ void scale_adjoint_kernel(float* __restrict__ g, size_t count, const double* __restrict__ multiplier) {
    const double m = *multiplier;
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x)
        g[i] = m == 0 ? 0.0f : float(g[i] * m);
}

void launch_scale_adjoint(Device& d, const Plan& p, float* g, const double* multiplier) {
    const size_t count = p.columns() * p.net->neurons.back();
    const int blocks = int(std::min<size_t>((count + 255) / 256, 1024));
    hipLaunchKernelGGL(scale_adjoint_kernel, blocks, 256, 0, d.stream, g, count, multiplier);
    HIP_CHECK(hipGetLastError());
}

// Gradient statistics (cuda/reduction_kernels.cuh:81-98): promote before squaring.
__device__ __forceinline__ GradStats combine_grad(GradStats a, const GradStats& b) {
    a.squared_norm += b.squared_norm;
    if (b.max_abs > a.max_abs) a.max_abs = b.max_abs;
    a.nonfinite += b.nonfinite;
    if (b.first < a.first) a.first = b.first;
    return a;
}

constexpr int kGradThreads = 1024;

__device__ GradStats block_reduce_grad(GradStats v) {
    __shared__ GradStats waves[kGradThreads / 64];
    for (int off = 32; off > 0; off >>= 1) {
        GradStats o;
        o.squared_norm = __shfl_down(v.squared_norm, off, 64);
        o.max_abs = __shfl_down(v.max_abs, off, 64);
        o.nonfinite = __shfl_down(v.nonfinite, off, 64);
        o.first = __shfl_down(v.first, off, 64);
        v = combine_grad(v, o);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) waves[wave] = v;
    __syncthreads();
    GradStats r{0.0, 0.0, 0ull, INT_MAX, 0};
    if (threadIdx.x == 0)
        for (int w = 0; w < kGradThreads / 64; ++w) r = combine_grad(r, waves[w]);
    return r;
}

// Statistics of several transitions' gradients in one launch (a host round
// trip per launch is what an epoch of small costs waits on): block t strides
// transition t's entries with 1,024 lanes, each lane in index order, then the
// fixed block reduction -- one order whatever the scheduling.
struct GradGroupArgs {
    const float* g[kMaxTransitions];
    int count[kMaxTransitions];
    int transitions;
};


// Entries are loaded eight at a time per lane (an index past the end reads the
// last entry again and is not counted), so that a transition of up to 8,192
// entries waits on one round of loads.
__global__ __launch_bounds__(kGradThreads) void grad_stats_kernel(GradGroupArgs a, GradStats* __restrict__ totals) {
    constexpr int U = 8;
    const int t = blockIdx.x, count = a.count[t];
    const float* __restrict__ g = a.g[t];
    GradStats acc{0.0, 0.0, 0ull, INT_MAX, 0};
    for (int i0 = threadIdx.x; i0 < count; i0 += U * kGradThreads) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = g[min(i0 + u * kGradThreads, count - 1)];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + u * kGradThreads;
            if (i >= count) break;
            const double v = x[u];
            if (!isfinite(v)) {
                ++acc.nonfinite;
                if (i < acc.first) acc.first = i;
            } else {
                acc.squared_norm += v * v;
                const double mag = fabs(v);
                if (mag > acc.max_abs) acc.max_abs = mag;
            }
        }
    }
    acc = block_reduce_grad(acc);
    if (threadIdx.x == 0) totals[t] = acc;
}

void launch_grad_stats(Device& d, const float* const* g, const int* counts, int transitions, int first_slot) {
    GradGroupArgs a{};
    a.transitions = transitions;
    for (int t = 0; t < transitions; ++t) {
        a.g[t] = g[t];
        a.count[t] = counts[t];
    }
    hipLaunchKernelGGL(grad_stats_kernel, transitions, kGradThreads, 0, d.stream, a, d.grad_totals + first_slot);
    HIP_CHECK(hipGetLastError());
}

// Row-major copies WT[i + n_in*o] = W[o + n_out*i] of several weight blocks in
// one launch (the network-fused backward's product operands).
struct TransposeArgs {
    const float* W[kMaxTransitions];
    float* WT[kMaxTransitions];
    int n_in[kMaxTransitions], n_out[kMaxTransitions];
    int begin[kMaxTransitions + 1];
    int transitions;
};

__global__ void transpose_kernel(TransposeArgs a) {
    const int total = a.begin[a.transitions];
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += blockDim.x * gridDim.x) {
        int t = 0;
        while (t + 1 < a.transitions && e >= a.begin[t + 1]) ++t;
        const int local = e - a.begin[t], ni = a.n_in[t];
        const int o = local / ni, i = local - o * ni;
        a.WT[t][local] = a.W[t][o + a.n_out[t] * i];
    }
}

void launch_transpose(Device& d, const float* const* W, float* const* WT, const int* n_in, const int* n_out,
                      int count) {
    for (int first = 0; first < count; first += kMaxTransitions) {
        TransposeArgs a{};
        a.transitions = std::min(kMaxTransitions, count - first);
        a.begin[0] = 0;
        for (int k = 0; k < a.transitions; ++k) {
            a.W[k] = W[first + k];
            a.WT[k] = WT[first + k];
            a.n_in[k] = n_in[first + k];
            a.n_out[k] = n_out[first + k];
            a.begin[k + 1] = a.begin[k] + n_in[first + k] * n_out[first + k];
        }
        if (!a.begin[a.transitions]) continue;
        const int blocks = std::max(1, std::min(1024, (a.begin[a.transitions] + 255) / 256));
        hipLaunchKernelGGL(transpose_kernel, blocks, 256, 0, d.stream, a);
        HIP_CHECK(hipGetLastError());
    }
}

// value into several buffers in one launch (buffer t holds begin[t+1]-begin[t] floats)
struct FillArgs {
    float* p[kMaxTransitions];
    int begin[kMaxTransitions + 1];
    int transitions;
};

__global__ void fill_grouped_kernel(FillArgs a, float value) {
    const int total = a.begin[a.transitions];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += blockDim.x * gridDim.x) {
        int t = 0;
        while (t + 1 < a.transitions && i >= a.begin[t + 1]) ++t;
        a.p[t][i - a.begin[t]] = value;
    }
}

void launch_fill_grouped(Device& d, float* const* p, const int* counts, int buffers, float value) {
    for (int first = 0; first < buffers; first += kMaxTransitions) {
        FillArgs a{};
        a.transitions = std::min(kMaxTransitions, buffers - first);
        a.begin[0] = 0;
        for (int k = 0; k < a.transitions; ++k) {
            a.p[k] = p[first + k];
            a.begin[k + 1] = a.begin[k] + counts[first + k];
        }
        if (!a.begin[a.transitions]) continue;
        const int blocks = std::max(1, std::min(1024, (a.begin[a.transitions] + 255) / 256));
        hipLaunchKernelGGL(fill_grouped_kernel, blocks, 256, 0, d.stream, a, value);
        HIP_CHECK(hipGetLastError());
    }
}

__global__ void fill_kernel(float* __restrict__ p, size_t count, float value) {
    for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x)
        p[i] = value;
}

void launch_fill(Device& d, float* p, size_t count, float value) {
    if (!count) return;
    const int blocks = int(std::min<size_t>((count + 255) / 256, 1024));
    hipLaunchKernelGGL(fill_kernel, blocks, 256, 0, d.stream, p, count, value);
    HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------------------------------------
// Optimizer launches (OptimizerArgs and the RPROP update are defined with the reductions).
// Entry j of transition t for this lane: each block lies within one
// transition, so t and its pointers are uniform (scalar loads).
__device__ __forceinline__ bool entry_of(const OptimizerArgs& a, int& t, int& j) {
    t = group_of(a.block_begin, a.transitions, int(blockIdx.x));
    j = (int(blockIdx.x) - a.block_begin[t]) * kOptimizerThreads + int(threadIdx.x);
    return j < a.begin[t + 1] - a.begin[t];
}

// One lane per entry: the gradient already reduced into the active buffer.
// The entry (state and gradient) is loaded first, so that its latency overlaps
// the publish copy's and the rule's.
__global__ __launch_bounds__(kOptimizerThreads) void rprop_kernel(OptimizerArgs a) {
    int t, j;
    const bool mine = entry_of(a, t, j);
    RpropState e{};
    float g = 0.0f;
    if (mine) {
        e = rprop_state(a, t, j);
        g = a.Ga[t][j];
    }
    publish_scalars(a);
    const bool finite = !a.test || test_gradients(a);
    if (!update_applies(a, finite)) return;
    if (mine) rprop_update(a, t, j, g, e);
}

// ADAM_k (cuda/derivative_kernels_v4.cu:780-799); M in S, V in the inactive buffer.
__global__ __launch_bounds__(kOptimizerThreads) void adam_kernel(OptimizerArgs a, float lr, float beta1, float beta2,
                                                                  float beta1t, float beta2t) {
#pragma clang fp contract(off)
    int t, j;
    const bool mine = entry_of(a, t, j);
    float g = 0.0f, m = 0.0f, v = 0.0f, w = 0.0f;
    if (mine) {  // loaded first, as in rprop_kernel
        g = a.Ga[t][j];
        m = a.S[t][j];
        v = a.Gi[t][j];
        w = a.W[t][j];
    }
    publish_scalars(a);
    const bool finite = !a.test || test_gradients(a);
    if (!update_applies(a, finite)) return;
    if (mine) {
        m = beta1 * m + (1 - beta1) * g;
        v = beta2 * v + (1 - beta2) * g * g;
        a.S[t][j] = m;
        a.Gi[t][j] = v;
        const float mh = m / (1 - beta1t), vh = v / (1 - beta2t);
        const float nW = float(double(w) - double(lr * mh) / (double(sqrtf(vh)) + 1e-8));
        const float kept = fabsf(nW) <= 20.0f ? nW : w;
        a.W[t][j] = kept;
        copy_transposed(a, t, j, kept);
    }
}

// Set_Resile_k / Reset_Resile_k (cuda/derivative_kernels_v4.cu:801-832).
__global__ __launch_bounds__(kOptimizerThreads) void steps_kernel(OptimizerArgs a, float value, int floor_mode) {
    int t, j;
    if (entry_of(a, t, j)) {
        if (!floor_mode || a.S[t][j] < value) {
            a.S[t][j] = value;
            a.Ga[t][j] = 0.0f;
            a.Gi[t][j] = 0.0f;
        }
    }
}

template <class F>
static void for_transition_groups(Net& net, F launch) {
    const int T = net.layers - 1;
    for (int first = 0; first < T; first += kMaxTransitions) {
        OptimizerArgs a{};
        a.transitions = std::min(kMaxTransitions, T - first);
        a.begin[0] = 0;
        a.block_begin[0] = 0;
        for (int k = 0; k < a.transitions; ++k) {
            const int t = first + k;
            const int act = net.active[t], inact = act == 1 ? 2 : 1;
            a.W[k] = net.state[0][t];
            a.S[k] = net.state[3][t];
            a.Ga[k] = net.state[act][t];
            a.Gi[k] = net.state[inact][t];
            a.WT[k] = net.wt[t];
            a.NO[k] = net.neurons[t + 1];
            a.NI[k] = net.neurons[t];
            a.begin[k + 1] = a.begin[k] + net.param_count(t);
            a.block_begin[k + 1] = a.block_begin[k] + (net.param_count(t) + kOptimizerThreads - 1) / kOptimizerThreads;
        }
        launch(a, a.block_begin[a.transitions]);
    }
}

// The first group's launch publishes `publish` (device scalar block, host
// mirror, bytes) when given.
static void set_publish(OptimizerArgs& a, const ScalarPublish* publish, bool& first) {
    if (!publish || !first) return;
    first = false;
    a.publish_src = static_cast<const unsigned*>(publish->src);
    a.publish_dst = static_cast<unsigned*>(publish->dst);
    a.publish_words = int(publish->bytes / sizeof(unsigned));
}

bool update_tests(const Net& net) {
    const int T = net.layers - 1;
    if (T > kMaxTransitions) return false;
    int chunks = 0;
    for (int t = 0; t < T; ++t) chunks += (net.param_count(t) + kOptimizerThreads - 1) / kOptimizerThreads;
    return chunks <= kTestChunks;
}

// The launch's own finiteness test over the group's active gradients, the
// totals written to the device's gradient slots (update_tests(net) holds:
// one transition group).
static void set_test(Device& d, OptimizerArgs& a, bool test) {
    if (!test) return;
    a.test = 1;
    a.stats = d.grad_totals;
}

void launch_rprop(Device& d, Net& net, const UpdateGuard* guard, const ScalarPublish* publish, bool test) {
    bool first = true;
    for_transition_groups(net, [&](OptimizerArgs a, int blocks) {
        if (guard) {
            a.guard = *guard;
            a.guarded = 1;
            a.verdict = d.update_verdict;
        }
        set_publish(a, publish, first);
        set_test(d, a, test);
        TraceScope trace(d, kTraceOptimizer, 28.0 * a.begin[a.transitions]);  // 4 reads, 3 writes per entry
        hipLaunchKernelGGL(rprop_kernel, blocks, kOptimizerThreads, 0, d.stream, a);
        HIP_CHECK(hipGetLastError());
    });
    if (guard) return;  // the caller switches the buffers once it knows whether the update applied
    for (auto& act : net.active) act = act == 1 ? 2 : 1;
    net.wt_current = true;
}

void launch_adam(Device& d, Net& net, int step, float lr, const UpdateGuard* guard, const ScalarPublish* publish,
                 bool test) {
    const float b1 = 0.9f, b2 = 0.999f;
    const float b1t = std::pow(b1, float(step)), b2t = std::pow(b2, float(step));
    bool first = true;
    for_transition_groups(net, [&](OptimizerArgs a, int blocks) {
        if (guard) {
            a.guard = *guard;
            a.guarded = 1;
            a.verdict = d.update_verdict;
        }
        set_publish(a, publish, first);
        set_test(d, a, test);
        hipLaunchKernelGGL(adam_kernel, blocks, kOptimizerThreads, 0, d.stream, a, lr, b1, b2, b1t, b2t);
        HIP_CHECK(hipGetLastError());
    });
    net.wt_current = true;
}

void launch_set_steps(Device& d, Net& net, float value) {
    for_transition_groups(net, [&](const OptimizerArgs& a, int blocks) {
        hipLaunchKernelGGL(steps_kernel, blocks, kOptimizerThreads, 0, d.stream, a, value, 0);
        HIP_CHECK(hipGetLastError());
    });
}

void launch_restore_steps(Device& d, Net& net, float floor_value) {
    for_transition_groups(net, [&](const OptimizerArgs& a, int blocks) {
        hipLaunchKernelGGL(steps_kernel, blocks, kOptimizerThreads, 0, d.stream, a, floor_value, 1);
        HIP_CHECK(hipGetLastError());
    });
}

// ------------------------------------------------------------------------------------------
// Scalar cost graph on one lane (cost_graph::execute, cuda/cost_graph.cuh:6-27;
// opcode semantics cuda/scalar_ops.cuh:5-26).
enum { kConstant, kLeaf, kField, kAdd, kSub, kMul, kDiv, kPower, kNeg, kExp, kLog, kSqrt, kSin, kCos, kTanh, kAttach };

__device__ double scalar_value(int op, double a, double b, double p) {
    switch (op) {
    case kConstant: return p;
    case kAdd: return a + b;
    case kSub: return a - b;
    case kMul: return a * b;
    case kDiv: return b == 0 ? NAN : a / b;
    case kPower: return ((a < 0 && floor(p) != p) || (a == 0 && p < 0)) ? NAN : pow(a, p);
    case kNeg: return -a;
    case kExp: return exp(a);
    case kLog: return a > 0 ? log(a) : NAN;
    case kSqrt: return a >= 0 ? sqrt(a) : NAN;
    case kSin: return sin(a);
    case kCos: return cos(a);
    case kTanh: return tanh(a);
    case kAttach: return a;
    default: return NAN;
    }
}

__device__ void scalar_partials(int op, double a, double b, double v, double p, double& da, double& db) {
    da = db = 0;
    switch (op) {
    case kAdd:
    case kAttach: da = db = 1; break;
    case kSub: da = 1; db = -1; break;
    case kMul: da = b; db = a; break;
    case kDiv: da = 1 / b; db = -v / b; break;
    case kPower: da = p == 0 ? 0 : (p == 1 ? 1 : p * pow(a, p - 1)); break;
    case kNeg: da = -1; break;
    case kExp: da = v; break;
    case kLog: da = 1 / a; break;
    case kSqrt: da = .5 / v; break;
    case kSin: da = cos(a); break;
    case kCos: da = -sin(a); break;
    case kTanh: da = 1 - v * v; break;
    default: break;
    }
}

__device__ void run_graph(const GraphLaunch& g) {
    const cpde_scalar_node* __restrict__ nodes = g.nodes;
    const CostStats* __restrict__ integrals = g.integrals;
    double *values = g.values, *adjoints = g.adjoints, *multipliers = g.multipliers;
    int* active = g.active;
    cpde_graph_summary* summary = g.summary;
    const int count = g.count, root = g.root, leaves = g.leaves;
    summary->bad_node = -1;
    summary->value = 0;
    for (int i = 0; i < leaves; ++i) multipliers[i] = 0;
    for (int i = 0; i < count; ++i) {
        const cpde_scalar_node n = nodes[i];
        adjoints[i] = 0;
        active[i] = n.op == kLeaf;
        if (n.op == kLeaf) values[i] = integrals[n.a].value;
        else {
            values[i] = scalar_value(n.op, n.a < 0 ? 0 : values[n.a], n.b < 0 ? 0 : values[n.b], n.parameter);
            if (n.op > 2) active[i] = active[n.a] || ((n.op <= kDiv || n.op == kAttach) && active[n.b]);
        }
        if (!isfinite(values[i]) && summary->bad_node < 0) summary->bad_node = i;
    }
    summary->value = values[root];
    if (!g.gradient || summary->bad_node >= 0) return;
    adjoints[root] = 1;
    for (int i = count - 1; i >= 0; --i) {
        const cpde_scalar_node n = nodes[i];
        const double seed = adjoints[i];
        if (seed == 0 || !active[i]) continue;
        if (n.op == kLeaf) multipliers[n.a] += seed;
        else if (n.op > 2) {
            double a, b;
            scalar_partials(n.op, values[n.a], n.b < 0 ? 0 : values[n.b], values[i], n.parameter, a, b);
            if (active[n.a]) adjoints[n.a] += seed * a;
            if ((n.op <= kDiv || n.op == kAttach) && active[n.b]) adjoints[n.b] += seed * b;
        }
        if (!isfinite(seed) && summary->bad_node < 0) summary->bad_node = i;
    }
    for (int i = 0; i < leaves; ++i)
        if (!isfinite(multipliers[i])) summary->bad_node = root;
}

// Graphs of at most this many nodes and leaves are evaluated on a copy in LDS.
constexpr int kGraphLdsNodes = 256, kGraphLdsLeaves = 64;

// run_graph with every lane of the block helping: the lanes copy the nodes and
// leaf values into LDS, lane 0 runs the same two sweeps on the copy (each step
// of the serial chain then waits on LDS, not on a round trip to global memory),
// and the lanes write the values, adjoints, activity, multipliers and summary
// out.  The same operations in the same order as run_graph, so the same bits.
// Larger graphs run on global memory.  Every lane of the block calls it.
// The LDS copy of a graph (graph_stage, graph_run): nodes {op, a, b, active},
// parameters, values, adjoints, leaf multipliers.
__shared__ int4 graph_node[kGraphLdsNodes];
__shared__ double graph_parameter[kGraphLdsNodes], graph_value[kGraphLdsNodes], graph_adjoint[kGraphLdsNodes];
__shared__ double graph_multiplier[kGraphLdsLeaves];
__shared__ int graph_bad_node;

__device__ __forceinline__ bool graph_in_lds(const GraphLaunch& g) {
    return g.count <= kGraphLdsNodes && g.leaves <= kGraphLdsLeaves;
}

// run_graph with every lane of the block helping, in two steps.  graph_stage:
// the lanes copy the nodes and the leaf values into LDS (no barrier; a launch
// that finishes costs first stages the graph before them, so the loads go out
// together).  graph_run: the totals the launch has just finished (fresh,
// finish_costs) replace their leaves' values, lane 0 runs the same two sweeps
// as run_graph on the copy (each step of the serial chain then waits on LDS,
// not on a round trip to global memory), and the lanes write the values,
// adjoints, activity, multipliers and summary out.  The same operations in the
// same order as run_graph, so the same bits.  Larger graphs run on global
// memory.  Every lane of the block (THREADS lanes) calls both.
template <int THREADS>
__device__ void graph_stage(const GraphLaunch& g) {
    if (!graph_in_lds(g)) return;
    for (int i = threadIdx.x; i < g.count; i += THREADS) {
        const cpde_scalar_node n = g.nodes[i];
        graph_node[i] = make_int4(n.op, n.a, n.b, n.op == kLeaf);
        graph_parameter[i] = n.parameter;
        graph_value[i] = n.op == kLeaf ? g.integrals[n.a].value : 0.0;
        graph_adjoint[i] = 0;
    }
    for (int i = threadIdx.x; i < g.leaves; i += THREADS) graph_multiplier[i] = 0;
}

template <int THREADS>
__device__ void graph_run(const GraphLaunch& g, bool fresh) {
    const int count = g.count, leaves = g.leaves, root = g.root;
    if (!graph_in_lds(g)) {
        if (threadIdx.x == 0) run_graph(g);
        return;
    }
    int4* const node = graph_node;
    double *const parameter = graph_parameter, *const value = graph_value, *const adjoint = graph_adjoint;
    double* const multiplier = graph_multiplier;
    __syncthreads();  // the staged copy is complete
    if (fresh) {
        const int finished = reduce_finished_count;
        for (int i = threadIdx.x; i < count; i += THREADS)
            if (node[i].x == kLeaf) {
                const CostStats* slot = g.integrals + node[i].y;
                for (int c = 0; c < finished; ++c)
                    if (reduce_finished_slot[c] == slot) value[i] = reduce_finished[c].value;
            }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        int bad = -1;
        for (int i = 0; i < count; ++i) {
            const int4 n = node[i];
            if (n.x != kLeaf) {
                value[i] = scalar_value(n.x, n.y < 0 ? 0 : value[n.y], n.z < 0 ? 0 : value[n.z], parameter[i]);
                if (n.x > 2) node[i].w = node[n.y].w || ((n.x <= kDiv || n.x == kAttach) && node[n.z].w);
            }
            if (!isfinite(value[i]) && bad < 0) bad = i;
        }
        if (g.gradient && bad < 0) {
            adjoint[root] = 1;
            for (int i = count - 1; i >= 0; --i) {
                const int4 n = node[i];
                const double seed = adjoint[i];
                if (seed == 0 || !n.w) continue;
                if (n.x == kLeaf) multiplier[n.y] += seed;
                else if (n.x > 2) {
                    double da, db;
                    scalar_partials(n.x, value[n.y], n.z < 0 ? 0 : value[n.z], value[i], parameter[i], da, db);
                    if (node[n.y].w) adjoint[n.y] += seed * da;
                    if ((n.x <= kDiv || n.x == kAttach) && node[n.z].w) adjoint[n.z] += seed * db;
                }
                if (!isfinite(seed) && bad < 0) bad = i;
            }
            for (int i = 0; i < leaves; ++i)
                if (!isfinite(multiplier[i])) bad = root;
        }
        graph_bad_node = bad;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < count; i += THREADS) {
        g.values[i] = value[i];
        g.adjoints[i] = adjoint[i];
        g.active[i] = node[i].w;
    }
    for (int i = threadIdx.x; i < leaves; i += THREADS) g.multipliers[i] = multiplier[i];
    if (threadIdx.x == 0) {
        g.summary->value = value[root];
        g.summary->bad_node = graph_bad_node;
    }
}

constexpr int kGraphThreads = 64;

__global__ __launch_bounds__(kGraphThreads) void graph_kernel(GraphLaunch g) {
    graph_stage<kGraphThreads>(g);
    graph_run<kGraphThreads>(g, false);
}

GraphLaunch graph_launch(Device& d, const cpde_scalar_node* nodes, int count, int root, int leaves, double* values,
                         double* adjoints, double* multipliers, int* active, cpde_graph_summary* summary,
                         bool gradient) {
    return GraphLaunch{nodes, d.cost_totals, values, adjoints, multipliers, active, summary,
                       count, root, leaves, int(gradient)};
}

void launch_graph(Device& d, const GraphLaunch& g) {
    hipLaunchKernelGGL(graph_kernel, 1, kGraphThreads, 0, d.stream, g);
    HIP_CHECK(hipGetLastError());
}

}  // namespace cpde
