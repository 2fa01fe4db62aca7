// Dense per-atom layers: fp32 MFMA GEMM with fused epilogues, RMSNorm rows,
// the Möbius element-head readout and the NEP per-element MLP.
#include <cmath>

#include "kernels.hpp"

namespace rune {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 64, kBN = 64, kBK = 16;

__device__ inline float act_f(int a, float x) {
    if (a == RUNE_ACT_SILU) return x / (1.0f + expf(-x));
    if (a == RUNE_ACT_TANH) return tanhf(x);
    if (a == RUNE_ACT_GELU) return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    if (a == kActSigmoid) return 1.0f / (1.0f + expf(-x));
    return x;
}

__device__ inline float act_d(int a, float x) {
    if (a == RUNE_ACT_SILU) {
        float s = 1.0f / (1.0f + expf(-x));
        return s * (1.0f + x * (1.0f - s));
    }
    if (a == RUNE_ACT_TANH) {
        float t = tanhf(x);
        return 1.0f - t * t;
    }
    if (a == RUNE_ACT_GELU)
        return 0.5f * (1.0f + erff(x * 0.70710678118654752f)) +
               x * expf(-0.5f * x * x) * 0.39894228040143268f;
    return 1.0f;
}

// 256 threads, 2x2 waves, each wave a 32x32 sub-tile of v_mfma_f32_16x16x4f32.
// MFMA operand layout: lane l supplies A[l%16][l/16] and B[l/16][l%16];
// accumulator register v of lane l is C[4*(l/16)+v][l%16].
__global__ void __launch_bounds__(256) k_gemm(int M, int N, int K, const float *__restrict__ A,
                                              int lda, const float *__restrict__ B, int ldb,
                                              float *__restrict__ C, int ldc, Epilogue ep) {
    __shared__ float As[kBK][kBM + 4];
    __shared__ float Bs[kBK][kBN + 4];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.x * kBM, n0 = blockIdx.y * kBN;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    floatx4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < K; k0 += kBK) {
#pragma unroll
        for (int it = 0; it < (kBM * kBK) / 256; ++it) {
            int idx = tid + 256 * it;
            int mm = idx / kBK, kk = idx % kBK;
            int gm = m0 + mm, gk = k0 + kk;
            As[kk][mm] = (gm < M && gk < K) ? A[size_t(gm) * lda + gk] : 0.0f;
        }
#pragma unroll
        for (int it = 0; it < (kBK * kBN) / 256; ++it) {
            int idx = tid + 256 * it;
            int kk = idx / kBN, nn = idx % kBN;
            int gk = k0 + kk, gn = n0 + nn;
            Bs[kk][nn] = (gk < K && gn < N) ? B[size_t(gk) * ldb + gn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 4) {
            int kq = kk + (lane >> 4), rr = lane & 15;
            float a0 = As[kq][wm + rr], a1 = As[kq][wm + 16 + rr];
            float b0 = Bs[kq][wn + rr], b1 = Bs[kq][wn + 16 + rr];
            acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                int row = m0 + wm + a * 16 + 4 * (lane >> 4) + v;
                int col = n0 + wn + b * 16 + (lane & 15);
                if (row >= M || col >= N) continue;
                float x = acc[a][b][v];
                if (ep.row_scale) x *= ep.row_scale[row];
                if (ep.bias) x += ep.bias[col];
                if (ep.emb) x += ep.emb[size_t(ep.types[row]) * ep.ld_emb + col];
                if (ep.residual) x += ep.residual[size_t(row) * ep.ldr + col];
#pragma unroll
                for (int k = 0; k < 3; ++k)
                    if (ep.gtab[k]) x += ep.gtab[k][size_t(ep.gidx[k][row]) * ep.gld[k] + col];
                if (ep.pre) ep.pre[size_t(row) * ep.ldp + col] = x;
                if (ep.act_split >= 0 && col >= ep.act_split)
                    x = act_f(ep.act2, x);
                else if (ep.act >= 0)
                    x = act_f(ep.act, x);
                if (ep.dact_from) x *= act_d(ep.dact, ep.dact_from[size_t(row) * ep.ldu + col]);
                C[size_t(row) * ldc + col] = x;
            }
        }
    }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__global__ void __launch_bounds__(256) k_row_inv_rms(int M, int N, const float *x, int ldx,
                                                     float eps, float *out) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    const float *p = x + size_t(row) * ldx;
    float s = 0.0f;
    for (int c = lane; c < N; c += 64) s += p[c] * p[c];
    s = wave_sum(s);
    if (lane == 0) out[row] = 1.0f / sqrtf(s / float(N) + eps);
}

__global__ void __launch_bounds__(256) k_rms_backward(int M, int N, const float *h, int ldh,
                                                      const float *inv_rms, const float *dz,
                                                      int ldz, const float *base, int ldb,
                                                      float *dh, int ldd) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    const float *hp = h + size_t(row) * ldh;
    const float *zp = dz + size_t(row) * ldz;
    float dot = 0.0f;
    for (int c = lane; c < N; c += 64) dot += zp[c] * hp[c];
    dot = wave_sum(dot);
    float r = inv_rms[row];
    float coef = r * r * r * dot / float(N);
    const float *bp = base ? base + size_t(row) * ldb : nullptr;
    float *dp = dh + size_t(row) * ldd;
    for (int c = lane; c < N; c += 64) {
        float v = r * zp[c] - coef * hp[c];
        dp[c] = bp ? bp[c] + v : v;
    }
}

__global__ void __launch_bounds__(256) k_readout(int M, int H, const float *h, int ldh,
                                                 const int32_t *types, const float *hw,
                                                 const float *hb, float eps, float *energies,
                                                 float *dh, int ldd) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    const float *hp = h + size_t(row) * ldh;
    const float *w = hw + size_t(types[row]) * H;
    float ss = 0.0f, dot = 0.0f;
    for (int c = lane; c < H; c += 64) {
        ss += hp[c] * hp[c];
        dot += hp[c] * w[c];
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    float r = 1.0f / sqrtf(ss / float(H) + eps);
    if (lane == 0) energies[row] = r * dot + hb[types[row]];
    if (dh) {
        float coef = r * r * r * dot / float(H);
        float *dp = dh + size_t(row) * ldd;
        for (int c = lane; c < H; c += 64) dp[c] = r * w[c] - coef * hp[c];
    }
}

__global__ void k_nep_mlp(int M, int Q, int Hn, const float *q, int ldq, const int32_t *types,
                          const float *w0, const float *b0, const float *w1, float shared_bias,
                          float *energies, float *dq, int want_grad) {
    int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= M) return;
    int t = types[row];
    const float *x = q + size_t(row) * ldq;
    const float *W0 = w0 + size_t(t) * Hn * Q;
    const float *B0 = b0 + size_t(t) * Hn;
    const float *W1 = w1 + size_t(t) * Hn;
    float e = 0.0f;
    float *g = want_grad ? dq + size_t(row) * ldq : nullptr;
    if (g)
        for (int k = 0; k < Q; ++k) g[k] = 0.0f;
    for (int h = 0; h < Hn; ++h) {
        float u = 0.0f;
        for (int k = 0; k < Q; ++k) u += W0[h * Q + k] * x[k];
        float a = tanhf(u + B0[h]);
        e += W1[h] * a;
        if (g) {
            float d = W1[h] * (1.0f - a * a);
            for (int k = 0; k < Q; ++k) g[k] += d * W0[h * Q + k];
        }
    }
    energies[row] = e - shared_bias;
}

}  // namespace

void gemm(int M, int N, int K, const float *A, int lda, const float *B, int ldb, float *C,
          int ldc, const Epilogue &ep, hipStream_t s) {
    if (M == 0 || N == 0) return;
    dim3 grid(ceil_div(M, kBM), ceil_div(N, kBN));
    hipLaunchKernelGGL(k_gemm, grid, dim3(256), 0, s, M, N, K, A, lda, B, ldb, C, ldc, ep);
    RUNE_HIP_CHECK(hipGetLastError());
}

void row_inv_rms(int M, int N, const float *x, int ldx, float eps, float *inv_rms, hipStream_t s) {
    if (M == 0) return;
    hipLaunchKernelGGL(k_row_inv_rms, dim3(ceil_div(M, 4)), dim3(256), 0, s, M, N, x, ldx, eps,
                       inv_rms);
    RUNE_HIP_CHECK(hipGetLastError());
}

void rms_backward(int M, int N, const float *h, int ldh, const float *inv_rms, const float *dz,
                  int ldz, const float *base, int ldb, float *dh, int ldd, hipStream_t s) {
    if (M == 0) return;
    hipLaunchKernelGGL(k_rms_backward, dim3(ceil_div(M, 4)), dim3(256), 0, s, M, N, h, ldh,
                       inv_rms, dz, ldz, base, ldb, dh, ldd);
    RUNE_HIP_CHECK(hipGetLastError());
}

void readout(int M, int H, const float *h, int ldh, const int32_t *types, const float *hw,
             const float *hb, float eps, float *energies, float *dh, int ldd, hipStream_t s) {
    if (M == 0) return;
    hipLaunchKernelGGL(k_readout, dim3(ceil_div(M, 4)), dim3(256), 0, s, M, H, h, ldh, types, hw,
                       hb, eps, energies, dh, ldd);
    RUNE_HIP_CHECK(hipGetLastError());
}

void nep_mlp(int M, int Q, int Hn, const float *q, int ldq, const int32_t *types,
             const float *w0, const float *b0, const float *w1, float shared_bias,
             float *energies, float *dq, int want_grad, hipStream_t s) {
    if (M == 0) return;
    hipLaunchKernelGGL(k_nep_mlp, dim3(ceil_div(M, 128)), dim3(128), 0, s, M, Q, Hn, q, ldq,
                       types, w0, b0, w1, shared_bias, energies, dq, want_grad);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
