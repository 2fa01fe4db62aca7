// Dense per-atom layers: fp32 MFMA GEMM with fused epilogues, RMSNorm rows,
// the Möbius element-head readout and the NEP per-element MLP.
#include <cmath>
#include <cstdlib>

#include "activation.hpp"
#include "kernels.hpp"

namespace rune {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// GEMM tiling: 4 waves in WMW x (4 / WMW), each wave (16*WM) x (16*WN) of the
// output; K advances kBK = 32 per LDS stage.
constexpr int kBK = 32, kLdk = kBK + 4;

// One K stage of a row-major operand X[rows, K] (A, or B stored as Bt[N, K])
// into registers.  Slot q of the tile covers row q/8 and four K values:
// vector path (ld % 4 == 0, 16-byte aligned base) k = 4*(q%8) + {0..3};
// scalar path k = q%8 + 8*{0..3}, so each load instruction stays coalesced.
// Either way the four values land in LDS columns 4*(q%8)..+3, and A and B use
// the same path, so LDS column c holds the same k for both operands.
template <int kRows, bool kVec>
__device__ inline void load_stage(float4 (&r)[kRows * 8 / 256], const float *__restrict__ X,
                                  int ld, int row0, int nrows, int k0, int K, int tid) {
#pragma unroll
    for (int it = 0; it < kRows * 8 / 256; ++it) {
        int q = tid + 256 * it, row = q >> 3, c4 = q & 7;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (row0 + row < nrows) {
            const float *x = X + size_t(row0 + row) * ld;
            if (kVec) {
                int k = k0 + 4 * c4;
                if (k + 3 < K) {
                    v = *reinterpret_cast<const float4 *>(x + k);
                } else if (k < K) {
                    v.x = x[k];
                    if (k + 1 < K) v.y = x[k + 1];
                    if (k + 2 < K) v.z = x[k + 2];
                }
            } else {
                int k = k0 + c4;
                if (k < K) v.x = x[k];
                if (k + 8 < K) v.y = x[k + 8];
                if (k + 16 < K) v.z = x[k + 16];
                if (k + 24 < K) v.w = x[k + 24];
            }
        }
        r[it] = v;
    }
}

// A full K stage (k0 + 32 <= K) of the vector path: no guards.  Rows past
// nrows read row nrows - 1 instead; their products land only in output rows
// or columns that the epilogue never stores.
template <int kRows>
__device__ inline void load_stage_full(float4 (&r)[kRows * 8 / 256], const float *__restrict__ X,
                                       int ld, int row0, int nrows, int k0, int tid) {
#pragma unroll
    for (int it = 0; it < kRows * 8 / 256; ++it) {
        int q = tid + 256 * it, row = min(row0 + (q >> 3), nrows - 1), c4 = q & 7;
        r[it] = *reinterpret_cast<const float4 *>(X + size_t(row) * ld + k0 + 4 * c4);
    }
}

template <int kRows>
__device__ inline void store_stage(const float4 (&r)[kRows * 8 / 256], float *S, int tid) {
#pragma unroll
    for (int it = 0; it < kRows * 8 / 256; ++it) {
        int q = tid + 256 * it;
        *reinterpret_cast<float4 *>(S + (q >> 3) * kLdk + 4 * (q & 7)) = r[it];
    }
}

// Epilogue straight from the accumulators: element (a, b, v) of this lane is
// row wm + 16a + 4g + v, column wn + 16b + rr of the tile (the MFMA output
// layout), so each store instruction writes 64-byte row segments and no LDS
// staging or block barrier is needed.  All loads of the terms come first (the
// stores to C cannot alias them then), in the order row scale, bias,
// embedding, residual, gathered rows; then the pre-activation store, the
// activation (act2 from column act_split on) and the activation derivative.
// Out-of-range elements load from clamped indices and store nothing.
// EK selects the activation at compile time for the common epilogues (the
// others keep the run-time choice): kEpiGate sigmoid before column act_split
// and tanh from it (the gate logits), kEpiSilu SiLU, kEpiDsilu the product
// with SiLU'(U) and no activation.
constexpr int kEpiAny = 0, kEpiGate = 1, kEpiSilu = 2, kEpiDsilu = 3;

template <int WM, int WN, int WMW, int EK = kEpiAny>
__device__ inline void tile_epilogue(floatx4 (&acc)[WM][WN], int M, int N,
                                     float *__restrict__ C, int ldc, const Epilogue &ep,
                                     int m0, int n0) {
    constexpr int WNW = 4 / WMW;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave / WNW) * 16 * WM, wn = (wave % WNW) * 16 * WN;
    const int g = lane >> 4, rr = lane & 15;
    float x[WM][4][WN], du[WM][4][WN];
#pragma unroll
    for (int a = 0; a < WM; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int rc = min(m0 + wm + 16 * a + 4 * g + v, M - 1);
            const float rs = ep.row_scale ? ep.row_scale[rc] : 1.0f;
            const int te = ep.emb ? ep.types[rc] : 0;
            int gi[3];
#pragma unroll
            for (int k = 0; k < 3; ++k) gi[k] = ep.gtab[k] ? ep.gidx[k][rc] : 0;
#pragma unroll
            for (int b = 0; b < WN; ++b) {
                const int cc = min(n0 + wn + 16 * b + rr, N - 1);
                float t = acc[a][b][v] * rs;
                if (ep.bias) t += ep.bias[cc];
                if (ep.emb) t += ep.emb[size_t(te) * ep.ld_emb + cc];
                if (ep.residual) t += ep.residual[size_t(rc) * ep.ldr + cc];
#pragma unroll
                for (int k = 0; k < 3; ++k)
                    if (ep.gtab[k]) t += ep.gtab[k][size_t(gi[k]) * ep.gld[k] + cc];
                x[a][v][b] = t;
                du[a][v][b] = ep.dact_from ? ep.dact_from[size_t(rc) * ep.ldu + cc] : 0.0f;
            }
        }
#pragma unroll
    for (int a = 0; a < WM; ++a)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = m0 + wm + 16 * a + 4 * g + v;
#pragma unroll
            for (int b = 0; b < WN; ++b) {
                const int col = n0 + wn + 16 * b + rr;
                if (row >= M || col >= N) continue;
                float t = x[a][v][b];
                if (ep.pre) ep.pre[size_t(row) * ep.ldp + col] = t;
                if constexpr (EK == kEpiGate) {
                    // tanh(t) = 2 sigmoid(2t) - 1: one logistic per element
                    const bool th = col >= ep.act_split;
                    const float sg = sigmoid_fast(th ? 2.0f * t : t);
                    t = th ? 2.0f * sg - 1.0f : sg;
                } else if constexpr (EK == kEpiSilu) {
                    t = t * sigmoid_fast(t);
                } else if constexpr (EK == kEpiDsilu) {
                    const float uu = du[a][v][b], sg = sigmoid_fast(uu);
                    t *= sg * (1.0f + uu * (1.0f - sg));
                } else {
                    if (ep.act_split >= 0 && col >= ep.act_split)
                        t = act_f(ep.act2, t);
                    else if (ep.act >= 0)
                        t = act_f(ep.act, t);
                    if (ep.dact_from) t *= act_d(ep.dact, du[a][v][b]);
                }
                C[size_t(row) * ldc + col] = t;
            }
        }
}

// C[M,N] = A[M,K] Bt[N,K]^T with the fused epilogue.  256 threads in WMW x
// (4 / WMW) waves, each (16*WM) x (16*WN) of the output.
// MFMA operand layout (v_mfma_f32_16x16x4f32): lane l supplies A[l%16][l/16]
// and B[l/16][l%16]; accumulator register v of lane l is C[4*(l/16)+v][l%16].
// The k index l/16 of MFMA step s in half h is LDS column 16h + 4(l/16) + s, so
// each lane fetches its four steps with one 16-byte LDS read.  Row stride
// kLdk = 36 floats keeps those reads free of bank conflicts.
// Tile t (the XCD-renumbered block) covers row tile t / nbn and column tile t % nbn.
// Batched launches (gridDim.y > 1) offset A, C by z times their batch strides
// and Bt by sb times z, or times L(z) - 1 (L the harmonic order of component z)
// when the batches share one weight block per order.
template <int WM, int WN, int WMW, bool kVec, bool kActA = false, int EK = kEpiAny>
__global__ void __launch_bounds__(256) k_gemm(int M, int N, int K, const float *__restrict__ A,
                                              int lda, const float *__restrict__ Bt, int ldb,
                                              float *__restrict__ C, int ldc, Epilogue ep,
                                              int nbn, GemmBatch bt) {
    if (gridDim.y > 1) {
        const int z = int(blockIdx.y);
        int w = z;
        if (bt.b_by_order) {
            w = 0;
            while ((w + 2) * (w + 2) - 1 <= z) ++w;
        }
        A += size_t(z) * bt.sa;
        C += size_t(z) * bt.sc;
        Bt += size_t(w) * bt.sb;
    }
    constexpr int WNW = 4 / WMW;
    constexpr int kBM = 16 * WM * WMW, BN = 16 * WN * WNW;
    __shared__ __attribute__((aligned(16))) float smem[(kBM + BN) * kLdk];
    float *As = smem, *Bs = smem + kBM * kLdk;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    // Blocks are dealt to the 8 XCDs round-robin; renumbering them so that each
    // XCD runs one contiguous range of tiles keeps all column tiles of a row
    // tile on one XCD, which then reads that A tile from HBM once.
    const int nb = int(gridDim.x), hx = int(blockIdx.x) & 7, hk = int(blockIdx.x) >> 3;
    const int tile = hx * (nb >> 3) + min(hx, nb & 7) + hk;
    const int m0 = (tile / nbn) * kBM, n0 = (tile % nbn) * BN;
    const int wm = (wave / WNW) * 16 * WM, wn = (wave % WNW) * 16 * WN;
    const int g = lane >> 4, rr = lane & 15;
    floatx4 acc[WM][WN];
#pragma unroll
    for (int a = 0; a < WM; ++a)
#pragma unroll
        for (int b = 0; b < WN; ++b) acc[a][b] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float4 ra[kBM * 8 / 256], rb[BN * 8 / 256];
    auto fetch = [&](int k0) {
        if (kVec && k0 + kBK <= K) {
            load_stage_full<kBM>(ra, A, lda, m0, M, k0, tid);
            load_stage_full<BN>(rb, Bt, ldb, n0, N, k0, tid);
        } else {
            load_stage<kBM, kVec>(ra, A, lda, m0, M, k0, K, tid);
            load_stage<BN, kVec>(rb, Bt, ldb, n0, N, k0, K, tid);
        }
    };
    fetch(0);
    for (int k0 = 0; k0 < K; k0 += kBK) {
        if constexpr (kActA) {
#pragma unroll
            for (int it = 0; it < kBM * 8 / 256; ++it)
                ra[it] = make_float4(act_f(ep.a_act, ra[it].x), act_f(ep.a_act, ra[it].y),
                                     act_f(ep.a_act, ra[it].z), act_f(ep.a_act, ra[it].w));
        }
        store_stage<kBM>(ra, As, tid);
        store_stage<BN>(rb, Bs, tid);
        __syncthreads();
        if (k0 + kBK < K) fetch(k0 + kBK);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float4 fa[WM], fb[WN];
#pragma unroll
            for (int a = 0; a < WM; ++a)
                fa[a] = *reinterpret_cast<const float4 *>(As + (wm + 16 * a + rr) * kLdk +
                                                          16 * h + 4 * g);
#pragma unroll
            for (int b = 0; b < WN; ++b)
                fb[b] = *reinterpret_cast<const float4 *>(Bs + (wn + 16 * b + rr) * kLdk +
                                                          16 * h + 4 * g);
#pragma unroll
            for (int a = 0; a < WM; ++a)
#pragma unroll
                for (int b = 0; b < WN; ++b) {
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a].x, fb[b].x, acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a].y, fb[b].y, acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a].z, fb[b].z, acc[a][b], 0, 0, 0);
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a].w, fb[b].w, acc[a][b], 0, 0, 0);
                }
        }
        __syncthreads();
    }
    tile_epilogue<WM, WN, WMW, EK>(acc, M, N, C, ldc, ep, m0, n0);
}

// One output element of the fused epilogue (the terms of tile_epilogue in the
// same order); the element's loads precede its stores, so C may alias an
// input element for element.
__device__ inline void epilogue_one(const Epilogue &ep, float acc, int row, int col,
                                    float *__restrict__ C, int ldc, float rms) {
    float t = acc;
    if (ep.rms_out)
        t *= rms;
    else if (ep.row_scale)
        t *= ep.row_scale[row];
    if (ep.bias) t += ep.bias[col];
    if (ep.emb) t += ep.emb[size_t(ep.types[row]) * ep.ld_emb + col];
    if (ep.residual) t += ep.residual[size_t(row) * ep.ldr + col];
#pragma unroll
    for (int k = 0; k < 3; ++k)
        if (ep.gtab[k]) t += ep.gtab[k][size_t(ep.gidx[k][row]) * ep.gld[k] + col];
    const float du = ep.dact_from ? ep.dact_from[size_t(row) * ep.ldu + col] : 0.0f;
    if (ep.pre) ep.pre[size_t(row) * ep.ldp + col] = t;
    if (ep.act_split >= 0 && col >= ep.act_split)
        t = act_f(ep.act2, t);
    else if (ep.act >= 0)
        t = act_f(ep.act, t);
    if (ep.dact_from) t *= act_d(ep.dact, du);
    C[size_t(row) * ldc + col] = t;
}

// Four consecutive K values x[k..k+3] of one operand row, zero past K.
template <bool kVec>
__device__ inline float4 load_k4(const float *__restrict__ x, int k, int K) {
    if (kVec && k + 3 < K) return *reinterpret_cast<const float4 *>(x + k);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (k < K) v.x = x[k];
    if (k + 1 < K) v.y = x[k + 1];
    if (k + 2 < K) v.z = x[k + 2];
    if (k + 3 < K) v.w = x[k + 3];
    return v;
}

// GEMM for grids smaller than the chip (a few hundred rows, e.g. every dense
// layer of a 512-atom cell): one 16 x (16*WN) output tile per 256-thread
// block, so the launch has 4-16x more blocks than the 64-row tiles, and the
// K range split over the block's 4 waves in 16-deep steps (step s to wave
// s % 4).  Operands go straight from global memory into the MFMA layout
// (lane l holds row l%16 at k = 16 s + 4 (l/16) + {0..3}; the next step's
// operands are loaded before the current step's products); the 4 partial
// tiles are summed through LDS in wave order and the epilogue runs per
// element with consecutive threads on consecutive columns.
template <int WN, bool kVec, bool kRms = false>
__global__ void __launch_bounds__(256) k_gemm_small(int M, int N, int K,
                                                    const float *__restrict__ A, int lda,
                                                    const float *__restrict__ Bt, int ldb,
                                                    float *__restrict__ C, int ldc, Epilogue ep,
                                                    int nbn) {
    constexpr int TN = 16 * WN;
    __shared__ float part[4][16][TN + 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m0 = (int(blockIdx.x) / nbn) * 16, n0 = (int(blockIdx.x) % nbn) * TN;
    const int r = lane & 15, g = lane >> 4;
    const float *a = A + size_t(min(m0 + r, M - 1)) * lda;
    const float *b[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) b[j] = Bt + size_t(min(n0 + 16 * j + r, N - 1)) * ldb;
    floatx4 acc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const int steps = (K + 15) >> 4;
    float4 fa = make_float4(0.0f, 0.0f, 0.0f, 0.0f), fb[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) fb[j] = fa;
    if (wave < steps) {
        fa = load_k4<kVec>(a, 16 * wave + 4 * g, K);
#pragma unroll
        for (int j = 0; j < WN; ++j) fb[j] = load_k4<kVec>(b[j], 16 * wave + 4 * g, K);
    }
    float ss = 0.0f;   // sum of squares of the A values this lane loads (rms epilogue)
    for (int st = wave; st < steps; st += 4) {
        if constexpr (kRms) ss += ((fa.x * fa.x + fa.y * fa.y) + fa.z * fa.z) + fa.w * fa.w;
        float4 na = fa, nb[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) nb[j] = fb[j];
        if (st + 4 < steps) {
            na = load_k4<kVec>(a, 16 * (st + 4) + 4 * g, K);
#pragma unroll
            for (int j = 0; j < WN; ++j) nb[j] = load_k4<kVec>(b[j], 16 * (st + 4) + 4 * g, K);
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.x, fb[j].x, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.y, fb[j].y, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.z, fb[j].z, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.w, fb[j].w, acc[j], 0, 0, 0);
        }
        fa = na;
#pragma unroll
        for (int j = 0; j < WN; ++j) fb[j] = nb[j];
    }
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) part[wave][4 * g + v][16 * j + r] = acc[j][v];
    // lanes r, r + 16, r + 32, r + 48 of every wave load row r
    __shared__ float rsum[4][16];
    if constexpr (kRms) {
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (lane < 16) rsum[wave][lane] = ss;
    }
    __syncthreads();
    __shared__ float rms[16];
    if constexpr (kRms) {
        if (threadIdx.x < 16) {
            const int rr = threadIdx.x;
            const float v = ((rsum[0][rr] + rsum[1][rr]) + rsum[2][rr]) + rsum[3][rr];
            rms[rr] = 1.0f / sqrtf(v / float(K) + ep.rms_eps);
            if (n0 == 0 && m0 + rr < M) ep.rms_out[m0 + rr] = rms[rr];
        }
        __syncthreads();
    }
    for (int e = threadIdx.x; e < 16 * TN; e += 256) {
        const int rr = e / TN, cc = e % TN, row = m0 + rr, col = n0 + cc;
        if (row >= M || col >= N) continue;
        const float v = ((part[0][rr][cc] + part[1][rr][cc]) + part[2][rr][cc]) + part[3][rr][cc];
        epilogue_one(ep, v, row, col, C, ldc, kRms ? rms[rr] : 1.0f);
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

// NEP per-element MLP, one wave per atom (4 per block): the atom's q row is
// staged in LDS; lane h computes hidden unit h (u = sum_k W0[h, k] q_k,
// a = tanh(u + b0)), the energy is the wave sum of W1[h] a_h, and for the
// gradient lane k forms dq_k = sum_h W1[h] (1 - a_h^2) W0[h, k] from the
// per-unit factors in LDS.
__global__ void __launch_bounds__(256) k_nep_mlp(int M, int Q, int Hn, const float *q, int ldq,
                                                 const int32_t *types, const float *w0,
                                                 const float *b0, const float *w1,
                                                 float shared_bias, float *energies, float *dq,
                                                 int want_grad) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    const bool live = row < M;
    float *xs = lds + wave * (Q + Hn), *ds = xs + Q;
    const int t = live ? types[row] : 0;
    const float *W0 = w0 + size_t(t) * Hn * Q;
    const float *B0 = b0 + size_t(t) * Hn;
    const float *W1 = w1 + size_t(t) * Hn;
    if (live)
        for (int k = lane; k < Q; k += 64) xs[k] = q[size_t(row) * ldq + k];
    __syncthreads();
    float e = 0.0f;
    if (live)
        for (int h = lane; h < Hn; h += 64) {
            float u = 0.0f;
            for (int k = 0; k < Q; ++k) u += W0[h * Q + k] * xs[k];
            const float a = tanhf(u + B0[h]);
            e += W1[h] * a;
            ds[h] = W1[h] * (1.0f - a * a);
        }
    e = wave_sum(e);
    __syncthreads();
    if (!live) return;
    if (lane == 0) energies[row] = e - shared_bias;
    if (want_grad)
        for (int k = lane; k < Q; k += 64) {
            float g = 0.0f;
            for (int h = 0; h < Hn; ++h) g += ds[h] * W0[h * Q + k];
            dq[size_t(row) * ldq + k] = g;
        }
}

}  // namespace

// Block tiles are 64 rows by 64 or 32 columns: narrow tiles keep each wave
// at 16-32 accumulator rows and 4-7 waves per SIMD, which hides the operand
// and epilogue latency better than wide tiles (measured on the per-record
// GEMMs: 64x64 / 64x32 beat 64x192 / 64x288 by 15-25 %).  The 32-column
// tile is taken when it pads N less.
static bool narrow_tile(int N) { return ceil_div(N, 32) * 32 < ceil_div(N, 64) * 64; }

// Below this many 64-row tiles (one per CU) a launch cannot fill the chip and
// the small-grid kernel, with K split over the waves of a block, is used.
constexpr int64_t kSmallGemmBlocks = 256;
// Rows from which a product takes the 64x96 tile (see gemm_any); the
// environment variable RUNE_TALL_ROWS overrides it (tests run that tile on
// small systems with it).
constexpr int64_t kTallRows = 2000000;
static int64_t tall_rows() {
    const char *v = std::getenv("RUNE_TALL_ROWS");
    return v && *v ? std::max<int64_t>(1, std::atoll(v)) : kTallRows;
}

template <int WM, int WN, int WMW = 2>
static void launch_gemm(bool vec, int M, int N, int K, const float *A, int lda, const float *Bt,
                        int ldb, float *C, int ldc, const Epilogue &ep, const GemmBatch &bt,
                        hipStream_t s) {
    constexpr int kBM = 16 * WM * WMW, BN = 16 * WN * (4 / WMW);
    int nbn = ceil_div(N, BN);
    int64_t blocks = int64_t(ceil_div(M, kBM)) * nbn;
    if (blocks > 0x7fffffff || bt.count > 65535)
        throw Error(RUNE_ERR_ARGUMENT, "gemm: problem too large");
    const dim3 grid(unsigned(blocks), unsigned(bt.count));
    // compile-time activation for the common epilogues (vector operands,
    // activation not applied to A)
    int ek = kEpiAny;
    if (ep.a_act < 0 && vec) {
        if (ep.act == kActSigmoid && ep.act_split >= 0 && ep.act2 == RUNE_ACT_TANH &&
            !ep.dact_from)
            ek = kEpiGate;
        else if (ep.act == RUNE_ACT_SILU && ep.act_split < 0 && !ep.dact_from)
            ek = kEpiSilu;
        else if (ep.act < 0 && ep.act_split < 0 && ep.dact_from && ep.dact == RUNE_ACT_SILU)
            ek = kEpiDsilu;
    }
    if (ek == kEpiGate)
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, true, false, kEpiGate>), grid, dim3(256), 0, s,
                           M, N, K, A, lda, Bt, ldb, C, ldc, ep, nbn, bt);
    else if (ek == kEpiSilu)
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, true, false, kEpiSilu>), grid, dim3(256), 0, s,
                           M, N, K, A, lda, Bt, ldb, C, ldc, ep, nbn, bt);
    else if (ek == kEpiDsilu)
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, true, false, kEpiDsilu>), grid, dim3(256), 0, s,
                           M, N, K, A, lda, Bt, ldb, C, ldc, ep, nbn, bt);
    else if (vec && ep.a_act >= 0)
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, true, true>), grid, dim3(256), 0, s, M, N, K, A,
                           lda, Bt, ldb, C, ldc, ep, nbn, bt);
    else if (ep.a_act >= 0)
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, false, true>), grid, dim3(256), 0, s, M, N, K, A,
                           lda, Bt, ldb, C, ldc, ep, nbn, bt);
    else if (vec)
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, true>), grid, dim3(256), 0, s, M, N, K, A, lda, Bt,
                           ldb, C, ldc, ep, nbn, bt);
    else
        hipLaunchKernelGGL((k_gemm<WM, WN, WMW, false>), grid, dim3(256), 0, s, M, N, K, A, lda,
                           Bt, ldb, C, ldc, ep, nbn, bt);
}

static void gemm_any(int M, int N, int K, const float *A, int lda, const float *Bt, int ldb,
                     float *C, int ldc, const Epilogue &ep, const GemmBatch &bt, hipStream_t s) {
    if (M == 0 || N == 0 || bt.count == 0) return;
    if (ep.rms_out && (ep.a_act >= 0 || bt.count != 1 || ep.row_scale))
        throw Error(RUNE_ERR_ARGUMENT, "gemm: the rms epilogue takes a plain single product");
    bool vec = lda % 4 == 0 && ldb % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
               (reinterpret_cast<uintptr_t>(Bt) & 15) == 0 && bt.sa % 4 == 0 && bt.sb % 4 == 0;
    const int64_t big_blocks = int64_t(ceil_div(M, 64)) * ceil_div(N, narrow_tile(N) ? 32 : 64);
    if (big_blocks < kSmallGemmBlocks && bt.count == 1 && ep.a_act < 0) {
        // 16 x 32 tiles, or 16 x 16 when that pads N less
        const bool n16 = ceil_div(N, 16) * 16 < ceil_div(N, 32) * 32;
        const int nbn = ceil_div(N, n16 ? 16 : 32);
        const dim3 grid(unsigned(int64_t(ceil_div(M, 16)) * nbn));
        if (ep.rms_out && n16 && vec)
            hipLaunchKernelGGL((k_gemm_small<1, true, true>), grid, dim3(256), 0, s, M, N, K, A,
                               lda, Bt, ldb, C, ldc, ep, nbn);
        else if (ep.rms_out && n16)
            hipLaunchKernelGGL((k_gemm_small<1, false, true>), grid, dim3(256), 0, s, M, N, K, A,
                               lda, Bt, ldb, C, ldc, ep, nbn);
        else if (ep.rms_out && vec)
            hipLaunchKernelGGL((k_gemm_small<2, true, true>), grid, dim3(256), 0, s, M, N, K, A,
                               lda, Bt, ldb, C, ldc, ep, nbn);
        else if (ep.rms_out)
            hipLaunchKernelGGL((k_gemm_small<2, false, true>), grid, dim3(256), 0, s, M, N, K, A,
                               lda, Bt, ldb, C, ldc, ep, nbn);
        else if (n16 && vec)
            hipLaunchKernelGGL((k_gemm_small<1, true>), grid, dim3(256), 0, s, M, N, K, A, lda, Bt,
                               ldb, C, ldc, ep, nbn);
        else if (n16)
            hipLaunchKernelGGL((k_gemm_small<1, false>), grid, dim3(256), 0, s, M, N, K, A, lda,
                               Bt, ldb, C, ldc, ep, nbn);
        else if (vec)
            hipLaunchKernelGGL((k_gemm_small<2, true>), grid, dim3(256), 0, s, M, N, K, A, lda, Bt,
                               ldb, C, ldc, ep, nbn);
        else
            hipLaunchKernelGGL((k_gemm_small<2, false>), grid, dim3(256), 0, s, M, N, K, A, lda,
                               Bt, ldb, C, ldc, ep, nbn);
    } else {
        // the row scales of the rms epilogue come from a row kernel here: the
        // 64-row tile kernels run slower with them folded in (more registers)
        Epilogue e = ep;
        if (ep.rms_out) {
            hipLaunchKernelGGL(k_row_inv_rms, dim3(ceil_div(M, 4)), dim3(256), 0, s, M, K, A, lda,
                               ep.rms_eps, ep.rms_out);
            e.row_scale = ep.rms_out;
            e.rms_out = nullptr;
        }
        // very tall products (the per-record GEMMs of large cells): 64x96
        // tiles (2 x 2 waves of 32 x 48) when they pad N no more than the
        // default tile, so a block does 1.5-3x the work behind one prologue
        // and epilogue (5 waves per SIMD; measured on C4, N = 264 / 192:
        // -0.9 / -0.3 ms per launch pair; 1 x 4 waves of 16 x 96 gained half
        // as much, 128 x 96 lost 4 ms; at 0.6 M rows no gain)
        const int pad = narrow_tile(N) ? ceil_div(N, 32) * 32 : ceil_div(N, 64) * 64;
        if (int64_t(M) >= tall_rows() && bt.count == 1 && N > 128 && ceil_div(N, 96) * 96 <= pad)
            launch_gemm<2, 3, 2>(vec, M, N, K, A, lda, Bt, ldb, C, ldc, e, bt, s);
        else if (narrow_tile(N))
            launch_gemm<1, 2, 4>(vec, M, N, K, A, lda, Bt, ldb, C, ldc, e, bt, s);
        else
            launch_gemm<2, 2, 2>(vec, M, N, K, A, lda, Bt, ldb, C, ldc, e, bt, s);
    }
    RUNE_HIP_CHECK(hipGetLastError());
}

void gemm(int M, int N, int K, const float *A, int lda, const float *Bt, int ldb, float *C,
          int ldc, const Epilogue &ep, hipStream_t s) {
    gemm_any(M, N, K, A, lda, Bt, ldb, C, ldc, ep, GemmBatch{}, s);
}

void gemm_batched(const GemmBatch &bt, int M, int N, int K, const float *A, int lda,
                  const float *Bt, int ldb, float *C, int ldc, hipStream_t s) {
    gemm_any(M, N, K, A, lda, Bt, ldb, C, ldc, Epilogue{}, bt, s);
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
    hipLaunchKernelGGL(k_nep_mlp, dim3(ceil_div(M, 4)), dim3(256),
                       sizeof(float) * 4 * size_t(Q + Hn), s, M, Q, Hn, q, ldq, types, w0, b0, w1,
                       shared_bias, energies, dq, want_grad);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
