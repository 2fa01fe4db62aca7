// EQ blocks: rune/mobius/equivariant.py (DirectionEncoder :12-39,
// EquivariantBlock :124-223) with the analytic reverse pass.
//
// Factored edge MLP.  The 673-wide edge input [rb | pair | C_c n_i | C_n n_j |
// probes_c | probes_n] is never formed: W_e[:, ctx_c] C_c and W_e[:, ctx_n] C_n
// are folded into per-atom projections A_i, B_j (one atom GEMM), the pair part
// into a [T*T, D] table, and the per-edge GEMM only sees [rb | probes_c |
// probes_n] (K = 17 + 2*lq*C).  A_i, B_j and the pair row are added in the
// GEMM epilogue by index.
//
// Angular states are stored [atom][channel][component] (components of order L
// at L*L-1 .. L*L+2L-1), matching direction[..., start:stop] of the reference.
#include <algorithm>
#include <cmath>

#include "activation.hpp"
#include "message.hpp"
#include "wave.hpp"

namespace rune {
namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;               // waves per block in the per-atom kernels
constexpr int kBlock = kWave * kWaves;
constexpr float kPi = 3.14159265358979323846f;

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ inline floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Copies n floats from global memory into this wave's LDS with up to eight
// loads per lane in flight (a plain strided loop would wait for each load
// before its LDS store and issue the next).
__device__ inline void stage_row(float *dst, const float *__restrict__ src, int n) {
    const int lane = threadIdx.x & (kWave - 1);
    for (int o = lane; o < n; o += 8 * kWave) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = src[min(o + u * kWave, n - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (o + u * kWave < n) dst[o + u * kWave] = v[u];
    }
}

__device__ __host__ inline int order_of(int k) {
    int L = 1;
    while ((L + 1) * (L + 1) - 1 <= k) ++L;
    return L;
}

struct EqArgs {
    Records r;
    int H, D, G, C, lq, nq, NG, NP, kb, na, nlm;
    int S;                    // records in flight per wave (lane slots of 64 / S lanes)
    int gmode;                // group-sum method of k_eq_pair_grp (3: k_eq_pair_grp_c)
    float eps, cutoff;
    const float *fc;          // [E]
    const float *tfc;         // [E] fc of transposed record t (fc[tidx[t]])
    const float *harm;        // [E, nq]
    const float *rb;          // [E, ldrb]
    int ldrb;
    const float *node;        // [N, NP] = A | B | V
    const float *dir_in;      // [N, C*nq]
    float *dir_out;           // [N, C*nq]
    const float *mixw;        // [lq, C, C]
    float *mixst;             // [N, C*nq] channel-mixed dir_in
    int act;                  // activation of the edge MLP
    int wlds;                 // LDS floats per wave of the edge-MLP kernels (multiple of 4)
    const int32_t *pair;      // [E] pair type index
    const float *pair_proj;   // [T*T, D]
    const float *wpc, *wpn;   // [lq*C, D] probe weights (neighbour side signed)
    const float *wrb;         // [kb, D] radial-basis weights
    int ldd;                  // row stride of ue, eh, due (a multiple of 64 DMC)
    float *ue, *eh;           // [E, D] edge MLP pre-activation, activation
    const float *ag;          // [E, NG] activated gates (sigmoid | tanh)
    float *msg, *rm, *uin;    // [N, H], [N], [N, H + lq*C]
    // reverse
    const float *duin;        // [N, H + lq*C]
    float *dmsg;              // [N, H]
    float *dht;               // [N, C*nq] dE/d(dir_out), total
    const float *ddir_out;    // [N, C*nq] from later blocks, or null
    float *dgg;               // [E, NG]
    float4 *dv;               // [E]
    float *dfc;               // [E] dE/dfc of the message terms, all blocks
    float *dy;                // [E, nq] dE/dY (both sides' shares, accumulated in turn)
    const float *dy_old;      // dy, or (first reverse block) a zero row: nothing to add to
    float *dnode;             // [N, NP]
    float *dmix;              // [N, C*nq]
    const float *due;         // [E, D]
    float *qbuf;              // [N, nq, 2 ldd] per-atom factors Qc | Qn of the block
    float *dqbuf;             // [N, nq, 2 ldd] their adjoints
    float *ddir_in;           // [N, C*nq]
};

// Direction encoder: out[i, c, k] = sum_n enc[(L(k)-1) C + c][n] s[i, n, k] scale[k].
// One atom per wave, four per block (blocks loop over atom groups); the
// block stages the projection weights, each wave its atom's moment row.
__global__ void __launch_bounds__(256) k_eq_encode(int N, const float *s, int na, int nlm,
                                                   const float *enc, const float *scale, int lq,
                                                   int C, int nq, int wrow, float *out) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
    float *W = lds;                                  // [lq C][na]
    float *row = lds + lq * C * na + wave * wrow;    // [na][nlm]
    for (int o = threadIdx.x; o < lq * C * na; o += blockDim.x) W[o] = enc[o];
    __syncthreads();
    // the next atom's moment row is loaded into registers while this one is
    // processed (rows of up to 4 floats per lane; longer rows are staged directly)
    const int RN = na * nlm, stride = int(gridDim.x) * 4;
    const bool pre = RN <= 4 * kWave;
    float pv[4];
    auto load_pre = [&](int i) {
#pragma unroll
        for (int u = 0; u < 4; ++u) pv[u] = s[size_t(i) * RN + min(lane + kWave * u, RN - 1)];
    };
    if (pre) load_pre(min(int(blockIdx.x) * 4 + wave, N - 1));
    for (int i = int(blockIdx.x) * 4 + wave; i < N; i += stride) {
        wave_sync();
        if (pre) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (lane + kWave * u < RN) row[lane + kWave * u] = pv[u];
            load_pre(min(i + stride, N - 1));
        } else {
            stage_row(row, s + size_t(i) * RN, RN);
        }
        wave_sync();
        for (int o = lane; o < C * nq; o += kWave) {
            const int c = o / nq, k = o - c * nq, L = order_of(k);
            const float *w = W + ((L - 1) * C + c) * na;
            float acc = 0.0f;
            for (int n = 0; n < na; ++n) acc += w[n] * (row[n * nlm + k] * scale[k]);
            out[size_t(i) * C * nq + o] = acc;
        }
    }
}

// Lane layout of the record loops: the wave holds S records at once, one per
// slot of W = 64 / S lanes.  Lane c of a slot owns channel c (c < C) with all
// NQ components of it (one contiguous state row), and the hidden / message
// columns c, c + W, c + 2W, ...
template <int S>
struct Lanes {
    static constexpr int W = kWave / S;
    static constexpr int HM = 4 * kWave / W;   // columns per lane for widths <= 256
    int lane, slot, c;
    bool act;
    __device__ explicit Lanes(int C) {
        lane = threadIdx.x & (kWave - 1);
        slot = lane / W;
        c = lane - slot * W;
        act = c < C;
    }
};

template <int NQ>
__device__ inline void load_row(float (&v)[NQ], const float *__restrict__ p) {
    if constexpr (NQ % 4 == 0) {
#pragma unroll
        for (int q = 0; q < NQ / 4; ++q) {
            const float4 t = reinterpret_cast<const float4 *>(p)[q];
            v[4 * q] = t.x;
            v[4 * q + 1] = t.y;
            v[4 * q + 2] = t.z;
            v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < NQ; ++k) v[k] = p[k];
    }
}

// Row r of a staged record array (row stride LY floats, 16-byte aligned rows
// when NQ % 4 == 0) into registers: 16-byte LDS reads at constant offsets.
template <int NQ, int LY>
__device__ inline void lds_row(float (&v)[NQ], const float *base, int r) {
    if constexpr (NQ % 4 == 0 && LY % 4 == 0) {
        const float4 *p = reinterpret_cast<const float4 *>(base + r * LY);
#pragma unroll
        for (int q = 0; q < NQ / 4; ++q) {
            const float4 t = p[q];
            v[4 * q] = t.x;
            v[4 * q + 1] = t.y;
            v[4 * q + 2] = t.z;
            v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < NQ; ++k) v[k] = base[r * LY + k];
    }
}

template <int NQ>
__device__ inline void store_row(const float (&v)[NQ], float *__restrict__ p) {
    if constexpr (NQ % 4 == 0) {
#pragma unroll
        for (int q = 0; q < NQ / 4; ++q)
            reinterpret_cast<float4 *>(p)[q] =
                make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else {
#pragma unroll
        for (int k = 0; k < NQ; ++k) p[k] = v[k];
    }
}

// out[n, c, k] = sum_c' W_L[c][c'] in[n, c', k] (trans = 0) or
// sum_c' W_L[c'][c] in[n, c', k] (trans = 1), L the order of component k,
// plus add[n, c, k] and add_t[n, k, c] when given.  One atom per wave (four
// per block, blocks loop over atom groups), on the matrix cores: for each
// order, out_L [C, 2L+1] = W_L [C, C] x in_L [C, 2L+1] as 16 x 16 tiles
// (channels padded to 16 MT, components to 16 per tile).  The W_L fragments stay in
// registers for the whole launch when they fit (MT <= 2), else the block
// stages them in LDS; the atom's input row is staged in the wave's LDS.
// MFMA operand layout as in k_eq_edge_adj: lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; accumulator v of lane l is C[4(l/16) + v][l%16].
template <int LQ, int MT>
__global__ void __launch_bounds__(256) k_eq_mix(int N, const float *mixw, const float *in, int C,
                                                int trans, const float *add, const float *add_t,
                                                float *out) {
    constexpr int NQ = LQ * (LQ + 2), KS = 4 * MT;   // k-steps over the padded channels
    constexpr bool kRegW = MT <= 2;
    extern __shared__ float lds[];
    const int CN = C * NQ, CNP = (CN + 3) & ~3, CP = 16 * MT;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
    float *row = lds + wave * 2 * CNP;               // this wave's input row [C][NQ]
    float *res = row + CNP;                          // and its result row [C][NQ]
    float *Wl = lds + 8 * CNP;                       // [LQ][CP][CP] as applied (MT > 2)
    auto wval = [&](int L, int c, int cc) {          // W_L[c][cc] as applied, 0 in the padding
        if (c >= C || cc >= C) return 0.0f;
        return trans ? mixw[size_t(L - 1) * C * C + size_t(cc) * C + c]
                     : mixw[size_t(L - 1) * C * C + size_t(c) * C + cc];
    };
    float Wr[kRegW ? LQ : 1][kRegW ? MT : 1][kRegW ? KS : 1];
    if constexpr (kRegW) {
#pragma unroll
        for (int L = 1; L <= LQ; ++L)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int s4 = 0; s4 < KS; ++s4) Wr[L - 1][mt][s4] = wval(L, 16 * mt + r, 4 * s4 + g);
    } else {
        for (int o = threadIdx.x; o < LQ * CP * CP; o += blockDim.x) {
            const int L = o / (CP * CP), q = o - L * CP * CP, c = q / CP, cc = q - c * CP;
            Wl[o] = wval(L + 1, c, cc);
        }
        __syncthreads();
    }
    // the next atom's input row is loaded into registers while this one is
    // processed (lane-strided floats, clamped so every lane loads)
    // (when a row is at most 16 floats per lane; wider rows are staged directly)
    constexpr int PF = (16 * MT * NQ + kWave - 1) / kWave;
    constexpr bool kPre = PF <= 16;
    const int stride = int(gridDim.x) * 4;
    float pre[kPre ? PF : 1];
    auto load_in = [&](int n) {
#pragma unroll
        for (int u = 0; u < (kPre ? PF : 1); ++u)
            pre[u] = in[size_t(n) * CN + min(lane + kWave * u, CN - 1)];
    };
    if constexpr (kPre) load_in(min(int(blockIdx.x) * 4 + wave, N - 1));
    for (int n = int(blockIdx.x) * 4 + wave; n < N; n += stride) {
        wave_sync();
        // rows move between HBM and LDS contiguously; add_t is transposed in LDS
        if constexpr (kPre) {
#pragma unroll
            for (int u = 0; u < PF; ++u)
                if (lane + kWave * u < CN) row[lane + kWave * u] = pre[u];
            load_in(min(n + stride, N - 1));
        } else {
            stage_row(row, in + size_t(n) * CN, CN);
        }
        if (add) {
            stage_row(res, add + size_t(n) * CN, CN);
        } else {
            for (int o = lane; o < CN; o += kWave) res[o] = 0.0f;
        }
        wave_sync();
        if (add_t) {
            for (int o = lane; o < CN; o += 4 * kWave) {
                float v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = add_t[size_t(n) * CN + min(o + u * kWave, CN - 1)];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int q = o + u * kWave;
                    if (q < CN) {
                        const int k = q / C, c = q - k * C;
                        res[c * NQ + k] += v[u];
                    }
                }
            }
            wave_sync();
        }
#pragma unroll
        for (int L = 1; L <= LQ; ++L) {
            const int st = L * L - 1, w = 2 * L + 1;
            // components of the order in tiles of 16 (two tiles at L = 8)
#pragma unroll
            for (int ct = 0; ct < (w + 15) / 16; ++ct) {
                const int kc = 16 * ct + r;
                floatx4 acc[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s4 = 0; s4 < KS; ++s4) {
                    const int cc = 4 * s4 + g;
                    const float b = (cc < C && kc < w) ? row[cc * NQ + st + min(kc, w - 1)] : 0.0f;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        float av;
                        if constexpr (kRegW)
                            av = Wr[L - 1][mt][s4];
                        else
                            av = Wl[(size_t(L - 1) * CP + 16 * mt + r) * CP + 4 * s4 + g];
                        acc[mt] = mfma4(av, b, acc[mt]);
                    }
                }
                if (kc < w) {
                    const int k = st + kc;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const int c = 16 * mt + 4 * g + v;
                            if (c < C) res[c * NQ + k] = acc[mt][v] + res[c * NQ + k];
                        }
                }
            }
        }
        wave_sync();
        for (int o = lane; o < CN; o += kWave) out[size_t(n) * CN + o] = res[o];
    }
}

__device__ inline int lane_get(int v, int q) { return __builtin_amdgcn_readlane(v, q); }
__device__ inline float lane_get(float v, int q) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), q));
}

// ---- factored edge MLP ----
// The probe columns of edge_mlp.0 act on p_c[L, c] = sum_m H_i[c, Lm] Y[Lm]
// and p_n[L, c] = (-1)^L sum_m H_j[c, Lm] Y[Lm] (equivariant.py:169-180).
// Contracting the channels first, W_pc p_c = sum_k Y[k] Qc_i[k, :] with
// Qc_i[k, d] = sum_c W_pc[d, (L(k), c)] H_i[c, k], and likewise Qn_j with
// the sign folded into the packed weights: NQ terms per record and output
// column instead of 2 LQ C.  The wave of an atom builds its Q in registers
// from its state row, so no per-record feature row is stored.
//
// Lanes own output columns d = d0 + lane + 64 u (u < DMC); a launch covers
// D in gridDim.y column blocks of 64 DMC, and the per-record [E, D] arrays
// have a row stride ldd that is a multiple of 64 DMC, so every lane loads and
// stores without a branch (loads of columns >= D read column D - 1, and the
// padding columns hold values nobody reads).  Branch-free loads keep the
// compiler's memory-counter waits exact, so prefetched loads stay in flight.

// Radial-basis weights held in registers; a longer basis reads the rest from L2.
constexpr int kRbRegs = 17;
constexpr int kRcStride = 20;   // LDS row of a record's radial basis when ldrb <= 20

template <int DMC>
struct EdgeCols {
    int d[DMC];    // owned column (store index, < ldd)
    int dl[DMC];   // clamped column (load index, < D)
    __device__ explicit EdgeCols(int D) {
        const int d0 = int(blockIdx.y) * kWave * DMC + int(threadIdx.x & (kWave - 1));
#pragma unroll
        for (int u = 0; u < DMC; ++u) {
            d[u] = d0 + kWave * u;
            dl[u] = min(d[u], D - 1);
        }
    }
};

// Q[k][u] = sum_c Hs[c, k] Wp[(L(k) - 1) C + c, dl[u]], Hs the atom's state
// row [C, NQ] staged in LDS.  The block's four waves stage the weights of one
// order at a time (this block's column chunk, [C][kWave * DMC]) into the
// shared Ws with one lane-parallel load, so the per-channel weight reads are
// LDS reads instead of a chain of dependent L2 loads.  Every wave of the
// block calls this (it holds block barriers); `active` is false for waves
// without an atom.
template <int LQ, int DMC>
__device__ inline void project_state(const float *Hs, const float *__restrict__ Wp, int C, int D,
                                     const int (&dl)[DMC], float (&Q)[LQ * (LQ + 2)][DMC],
                                     float *Ws, bool active) {
    constexpr int NQ = LQ * (LQ + 2), WC = kWave * DMC;
    const int c0 = int(blockIdx.y) * WC, cw = min(WC, D - c0);
#pragma unroll
    for (int k = 0; k < NQ; ++k)
#pragma unroll
        for (int u = 0; u < DMC; ++u) Q[k][u] = 0.0f;
#pragma unroll
    for (int L = 1; L <= LQ; ++L) {
        const int st = L * L - 1;
        const float *wl = Wp + size_t(L - 1) * C * D + c0;
        __syncthreads();
        for (int o = threadIdx.x; o < C * WC; o += 8 * kBlock) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int q = min(o + u * kBlock, C * WC - 1), c = q / WC, x = min(q - c * WC, cw - 1);
                v[u] = wl[size_t(c) * D + x];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (o + u * kBlock < C * WC) Ws[o + u * kBlock] = v[u];
        }
        __syncthreads();
        if (active) {
            for (int c = 0; c < C; ++c) {
                float w[DMC];
#pragma unroll
                for (int u = 0; u < DMC; ++u) w[u] = Ws[c * WC + dl[u] - c0];
#pragma unroll
                for (int m = 0; m < 2 * L + 1; ++m) {
                    const float h = Hs[c * NQ + st + m];
#pragma unroll
                    for (int u = 0; u < DMC; ++u) Q[st + m][u] += h * w[u];
                }
            }
        }
    }
    __syncthreads();
}

// Keeps the factor for the reverse pass: out[k * ld + d].
template <int LQ, int DMC>
__device__ inline void store_factor(const float (&Q)[LQ * (LQ + 2)][DMC], float *out, int ld,
                                    const int (&d)[DMC]) {
#pragma unroll
    for (int k = 0; k < LQ * (LQ + 2); ++k)
#pragma unroll
        for (int u = 0; u < DMC; ++u) out[size_t(k) * ld + d[u]] = Q[k][u];
}

// Harmonic row (and radial-basis row when R) of record e into the wave's LDS
// slot of lane q: every lane of the chunk loads (the rows of records with
// fc = 0 are finite and their results are discarded).
template <int NQ, int LY>
__device__ inline void stage_record(const EqArgs &a, int e, float *Yc, float *Rc, int q) {
    float y[NQ];
    load_row(y, a.harm + size_t(e) * NQ);
#pragma unroll
    for (int k = 0; k < NQ; ++k) Yc[q * LY + k] = y[k];
    if (Rc) {
        // rows of kRcStride floats (zero past ldrb) when the basis fits, so
        // the readers use constant offsets; else rows of ldrb
        const float4 *rb = reinterpret_cast<const float4 *>(a.rb + size_t(e) * a.ldrb);
        if (a.ldrb <= kRcStride) {
#pragma unroll
            for (int k = 0; k < kRcStride / 4; ++k)
                reinterpret_cast<float4 *>(Rc + q * kRcStride)[k] =
                    4 * k < a.ldrb ? rb[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        } else {
            for (int k = 0; k < a.ldrb / 4; ++k)
                reinterpret_cast<float4 *>(Rc + q * a.ldrb)[k] = rb[k];
        }
    }
}

// Neighbour side: for every record e that sees atom j as neighbour,
// ue[e, :] = B_j + pair_proj[pair_e] + (fc != 0: Qn_j Y_e + W_rb rb_e).  The
// harmonic and radial-basis rows of a chunk of 64 records are gathered into
// LDS with one lane-parallel load; the pair row (a small table) of the next
// record is loaded while the current one is computed.
template <int LQ, int DMC>
__global__ void __launch_bounds__(kBlock) k_eq_edge_nbr(EqArgs a) {
    constexpr int NQ = LQ * (LQ + 2), LY = NQ + (NQ % 4 == 0 ? 4 : 1);
    extern __shared__ float lds[];
    const int j = wave_atom(a.r);
    const int lane = threadIdx.x & (kWave - 1), C = a.C, D = a.D, CN = C * NQ, kb = a.kb;
    const int LR = a.ldrb, ldd = a.ldd, cn4 = (CN + 3) & ~3;
    const EdgeCols<DMC> col(D);
    float Q[NQ][DMC];
    {
        // prologue layout: the four state rows, then the shared weight chunk
        float *Hs = lds + (threadIdx.x >> 6) * cn4;
        if (j >= 0) stage_row(Hs, a.dir_in + size_t(j) * CN, CN);
        project_state<LQ, DMC>(Hs, a.wpn, C, D, col.dl, Q, lds + kWaves * cn4, j >= 0);
    }
    if (j < 0) return;
    float *Yc = lds + (threadIdx.x >> 6) * a.wlds;
    float *Rc = Yc + kWave * LY;
    store_factor<LQ, DMC>(Q, a.qbuf + size_t(j) * NQ * 2 * ldd + ldd, 2 * ldd, col.d);
    float wr[kRbRegs][DMC], Bj[DMC];
#pragma unroll
    for (int k = 0; k < kRbRegs; ++k)
#pragma unroll
        for (int u = 0; u < DMC; ++u)
            wr[k][u] = k < kb ? a.wrb[size_t(k) * D + col.dl[u]] : 0.0f;
#pragma unroll
    for (int u = 0; u < DMC; ++u) Bj[u] = a.node[size_t(j) * a.NP + D + col.dl[u]];
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    const bool fixed_rc = LR <= kRcStride;
    for (int t0 = tb; t0 < te; t0 += kWave) {
        const int cnt = min(kWave, te - t0);
        int me = 0, mp = 0;
        float mf = 0.0f;
        wave_sync();
        if (lane < cnt) {
            me = a.r.tidx[t0 + lane];
            mf = a.tfc[t0 + lane];
            mp = a.pair[me];
            stage_record<NQ, LY>(a, me, Yc, Rc, lane);
        }
        wave_sync();
        float P[DMC];
        {
            const int pr = lane_get(mp, 0);
#pragma unroll
            for (int u = 0; u < DMC; ++u) P[u] = a.pair_proj[size_t(pr) * D + col.dl[u]];
        }
        for (int q = 0; q < cnt; ++q) {
            float Pn[DMC];
            const int pr = lane_get(mp, min(q + 1, cnt - 1));
#pragma unroll
            for (int u = 0; u < DMC; ++u) Pn[u] = a.pair_proj[size_t(pr) * D + col.dl[u]];
            const int e = lane_get(me, q);
            float acc[DMC];
#pragma unroll
            for (int u = 0; u < DMC; ++u) acc[u] = 0.0f;
            if constexpr (NQ % 4 == 0) {
                // 16-byte rows (LY = NQ + 4), constant offsets
                const float4 *y4 = reinterpret_cast<const float4 *>(Yc + q * LY);
#pragma unroll
                for (int k4 = 0; k4 < NQ / 4; ++k4) {
                    const float4 y = y4[k4];
#pragma unroll
                    for (int u = 0; u < DMC; ++u) {
                        acc[u] += y.x * Q[4 * k4][u];
                        acc[u] += y.y * Q[4 * k4 + 1][u];
                        acc[u] += y.z * Q[4 * k4 + 2][u];
                        acc[u] += y.w * Q[4 * k4 + 3][u];
                    }
                }
            } else {
#pragma unroll
                for (int k = 0; k < NQ; ++k) {
                    const float y = Yc[q * LY + k];
#pragma unroll
                    for (int u = 0; u < DMC; ++u) acc[u] += y * Q[k][u];
                }
            }
            if (fixed_rc) {
                const float *rq = Rc + q * kRcStride;
#pragma unroll
                for (int k = 0; k < kRbRegs; ++k) {
                    const float r = rq[k];
#pragma unroll
                    for (int u = 0; u < DMC; ++u) acc[u] += r * wr[k][u];
                }
                for (int k = kRbRegs; k < kb; ++k) {
                    const float r = rq[k];
#pragma unroll
                    for (int u = 0; u < DMC; ++u)
                        acc[u] += r * a.wrb[size_t(k) * D + col.dl[u]];
                }
            } else {
#pragma unroll
                for (int k = 0; k < kRbRegs; ++k) {
                    const float r = Rc[q * LR + min(k, LR - 1)];
#pragma unroll
                    for (int u = 0; u < DMC; ++u) acc[u] += r * wr[k][u];
                }
                for (int k = kRbRegs; k < kb; ++k) {
                    const float r = Rc[q * LR + k];
#pragma unroll
                    for (int u = 0; u < DMC; ++u)
                        acc[u] += r * a.wrb[size_t(k) * D + col.dl[u]];
                }
            }
            const bool on = lane_get(mf, q) != 0.0f;
#pragma unroll
            for (int u = 0; u < DMC; ++u)
                a.ue[size_t(e) * ldd + col.d[u]] = (Bj[u] + P[u]) + (on ? acc[u] : 0.0f);
            copy(P, Pn);
        }
    }
}

// Centre side: u = A_i + (the neighbour pass's row) + (fc != 0: Qc_i Y_e),
// stored as ue (pre-activation) and eh = act(u).  The records of a centre are
// contiguous, so the rows of the next six are loaded while one is computed.
template <int LQ, int DMC>
__global__ void __launch_bounds__(kBlock) k_eq_edge_centre(EqArgs a) {
    constexpr int NQ = LQ * (LQ + 2), LY = NQ + (NQ % 4 == 0 ? 4 : 1);
    extern __shared__ float lds[];
    const int i = wave_atom(a.r);
    const int lane = threadIdx.x & (kWave - 1), C = a.C, D = a.D, CN = C * NQ, act = a.act;
    const int ldd = a.ldd, cn4 = (CN + 3) & ~3;
    const EdgeCols<DMC> col(D);
    float Q[NQ][DMC], A[DMC];
    {
        float *Hs = lds + (threadIdx.x >> 6) * cn4;
        if (i >= 0) stage_row(Hs, a.dir_in + size_t(i) * CN, CN);
        project_state<LQ, DMC>(Hs, a.wpc, C, D, col.dl, Q, lds + kWaves * cn4, i >= 0);
    }
    if (i < 0) return;
    float *Yc = lds + (threadIdx.x >> 6) * a.wlds;
    store_factor<LQ, DMC>(Q, a.qbuf + size_t(i) * NQ * 2 * ldd, 2 * ldd, col.d);
#pragma unroll
    for (int u = 0; u < DMC; ++u) A[u] = a.node[size_t(i) * a.NP + col.dl[u]];
    const int b0 = a.r.ptr[i], b1 = a.r.ptr[i + 1];
    if (b1 == b0) return;
    auto fetch = [&](int e, float (&X)[DMC]) {
        const size_t row = size_t(min(e, b1 - 1)) * ldd;
#pragma unroll
        for (int u = 0; u < DMC; ++u) X[u] = a.ue[row + col.d[u]];
    };
    // ring of the next kPf rows: loads stay in flight across the stores of
    // several records (vector loads and stores share one in-order counter)
    constexpr int kPf = 6;
    float X[kPf][DMC];
#pragma unroll
    for (int f = 0; f < kPf; ++f) fetch(b0 + f, X[f]);
    for (int t0 = b0; t0 < b1; t0 += kWave) {
        const int cnt = min(kWave, b1 - t0);
        float mf = 0.0f;
        wave_sync();
        if (lane < cnt) {
            mf = a.fc[t0 + lane];
            stage_record<NQ, LY>(a, t0 + lane, Yc, nullptr, lane);
        }
        wave_sync();
        for (int q = 0; q < cnt; ++q) {
            const int e = t0 + q;
            float Xn[DMC];
            fetch(e + kPf, Xn);
            float acc[DMC];
#pragma unroll
            for (int u = 0; u < DMC; ++u) acc[u] = 0.0f;
            {
                float y[NQ];
                lds_row<NQ, LY>(y, Yc, q);
#pragma unroll
                for (int k = 0; k < NQ; ++k)
#pragma unroll
                    for (int u = 0; u < DMC; ++u) acc[u] += y[k] * Q[k][u];
            }
            const bool on = lane_get(mf, q) != 0.0f;
            float v[DMC], h[DMC];
#pragma unroll
            for (int u = 0; u < DMC; ++u) v[u] = (A[u] + X[0][u]) + (on ? acc[u] : 0.0f);
            // one uniform branch per record for the activation (SiLU inline)
            if (act == RUNE_ACT_SILU) {
#pragma unroll
                for (int u = 0; u < DMC; ++u) h[u] = v[u] * sigmoid_fast(v[u]);
            } else {
#pragma unroll
                for (int u = 0; u < DMC; ++u) h[u] = act_f(act, v[u]);
            }
#pragma unroll
            for (int u = 0; u < DMC; ++u) {
                a.ue[size_t(e) * ldd + col.d[u]] = v[u];
                a.eh[size_t(e) * ldd + col.d[u]] = h[u];
            }
#pragma unroll
            for (int f = 0; f + 1 < kPf; ++f) copy(X[f], X[f + 1]);
            copy(X[kPf - 1], Xn);
        }
    }
}

// Messages and transported / injected direction states of centre i, then the
// update input [RMSNorm(msg) | per-(L, c) squared norms of dir_out].  The
// neighbour rows (mixed state, values) are gathered for S records at a time.
template <int LQ, int S>
__global__ void __launch_bounds__(kBlock, 2) k_eq_aggregate(EqArgs a) {
    constexpr int NQ = LQ * (LQ + 2), LY = NQ + (NQ % 4 == 0 ? 4 : 1);
    using Ln = Lanes<S>;
    constexpr int HM = Ln::HM;
    extern __shared__ float lds[];
    const int i = wave_atom(a.r);
    if (i < 0) return;
    const Ln ln(a.C);
    float *Yc = lds + (threadIdx.x >> 6) * kWave * LY;
    const int H = a.H, G = a.G, C = a.C, CN = C * NQ, LC = LQ * C, NG = a.NG;
    const int gw = H / G;
    const int e_begin = a.r.view[4 * i], e_end = a.r.view[4 * i + 1];
    float acc[NQ], macc[HM];
    zero(acc);
    zero(macc);
    for (int t0 = e_begin; t0 < e_end; t0 += kWave) {
        const int cnt = min(kWave, e_end - t0);
        int mj = 0;
        float mf = 0.0f;
        wave_sync();
        if (ln.lane < cnt) {
            mj = a.r.nbr[t0 + ln.lane];
            mf = a.fc[t0 + ln.lane];
            float y[NQ];
            load_row(y, a.harm + size_t(t0 + ln.lane) * NQ);
#pragma unroll
            for (int k = 0; k < NQ; ++k) Yc[ln.lane * LY + k] = y[k];
        }
        wave_sync();
        // every lane loads (clamped indices), so the compiler's waits stay exact
        auto fetch = [&](int q, float (&mx)[NQ], float (&tt)[LQ], float (&ti)[LQ],
                         float (&v)[HM], float (&g)[HM], float &f) {
            const int qq = min(q, cnt - 1);
            const int j = bcast(mj, qq);
            const float fq = bcast(mf, qq);   // every lane joins the shuffle
            f = q < cnt ? fq : 0.0f;
            const int e = t0 + qq, cl = min(ln.c, C - 1);
            load_row(mx, a.mixst + size_t(j) * CN + cl * NQ);
            const float *gd = a.ag + size_t(e) * NG + G + cl;
#pragma unroll
            for (int L = 0; L < LQ; ++L) {
                tt[L] = gd[L * C];
                ti[L] = gd[LC + L * C];
            }
            const float *Vr = a.node + size_t(j) * a.NP + 2 * a.D;
            const float *gr = a.ag + size_t(e) * NG;
#pragma unroll
            for (int u = 0; u < HM; ++u) {
                const int h = min(ln.c + Ln::W * u, H - 1);
                v[u] = Vr[h];
                g[u] = gr[h / gw];
            }
        };
        // two rounds of gathers in flight
        float M[NQ], tT[LQ], tI[LQ], V[HM], g[HM], fc;
        float M1[NQ], tT1[LQ], tI1[LQ], V1[HM], g1[HM], fc1;
        fetch(ln.slot, M, tT, tI, V, g, fc);
        fetch(ln.slot + S, M1, tT1, tI1, V1, g1, fc1);
        for (int q0 = 0; q0 < cnt; q0 += S) {
            float Mn[NQ], tTn[LQ], tIn[LQ], Vn[HM], gn[HM], fcn;
            fetch(q0 + 2 * S + ln.slot, Mn, tTn, tIn, Vn, gn, fcn);
            if (fc != 0.0f) {
                if (ln.act) {
                    float Y[NQ];
                    lds_row<NQ, LY>(Y, Yc, q0 + ln.slot);
#pragma unroll
                    for (int L = 1; L <= LQ; ++L)
#pragma unroll
                        for (int m = 0; m < 2 * L + 1; ++m) {
                            const int k = L * L - 1 + m;
                            acc[k] += fc * (tT[L - 1] * M[k] + tI[L - 1] * Y[k]);
                        }
                }
#pragma unroll
                for (int u = 0; u < HM; ++u) macc[u] += g[u] * fc * V[u];
            }
            copy(M, M1);
            copy(tT, tT1);
            copy(tI, tI1);
            copy(V, V1);
            copy(g, g1);
            fc = fc1;
            copy(M1, Mn);
            copy(tT1, tTn);
            copy(tI1, tIn);
            copy(V1, Vn);
            copy(g1, gn);
            fc1 = fcn;
        }
    }
    fold_slots<S>(acc);
    fold_slots<S>(macc);
    const int ldu = H + LC;
    if (ln.slot == 0 && ln.act) {
        float v[NQ];
        load_row(v, a.dir_in + size_t(i) * CN + ln.c * NQ);
#pragma unroll
        for (int k = 0; k < NQ; ++k) v[k] += acc[k];
        store_row(v, a.dir_out + size_t(i) * CN + ln.c * NQ);
#pragma unroll
        for (int L = 1; L <= LQ; ++L) {
            float s = 0.0f;
#pragma unroll
            for (int m = 0; m < 2 * L + 1; ++m) s += v[L * L - 1 + m] * v[L * L - 1 + m];
            a.uin[size_t(i) * ldu + H + (L - 1) * C + ln.c] = s;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < HM; ++u)
        if (ln.c + Ln::W * u < H) ss += macc[u] * macc[u];
    ss = group_sum(ss, Ln::W);
    const float r = 1.0f / sqrtf(ss / float(H) + a.eps);
    if (ln.lane == 0) a.rm[i] = r;
    if (ln.slot == 0) {
#pragma unroll
        for (int u = 0; u < HM; ++u) {
            const int h = ln.c + Ln::W * u;
            if (h < H) {
                a.msg[size_t(i) * H + h] = macc[u];
                a.uin[size_t(i) * ldu + h] = macc[u] * r;
            }
        }
    }
}

__global__ void __launch_bounds__(kWave) k_eq_node_backward(EqArgs a) {
    const int i = blockIdx.x, lane = threadIdx.x;
    const int H = a.H, C = a.C, nq = a.nq, LC = a.lq * C, ldu = H + LC, CN = C * nq;
    const float *d = a.duin + size_t(i) * ldu;
    const float *m = a.msg + size_t(i) * H;
    float dot = 0.0f;
#pragma unroll 4
    for (int c = lane; c < H; c += kWave) dot += d[c] * m[c];
    dot = wave_sum(dot);
    float r = a.rm[i];
    float coef = r * r * r * dot / float(H);
#pragma unroll 4
    for (int c = lane; c < H; c += kWave) a.dmsg[size_t(i) * H + c] = r * d[c] - coef * m[c];
#pragma unroll 4
    for (int o = lane; o < CN; o += kWave) {
        int c = o / nq, k = o - c * nq, L = order_of(k);
        float g = a.ddir_out ? a.ddir_out[size_t(i) * CN + o] : 0.0f;
        g += 2.0f * a.dir_out[size_t(i) * CN + o] * d[H + (L - 1) * C + c];
        a.dht[size_t(i) * CN + o] = g;
    }
}

__device__ inline float cutoff_slope(float d, float rc) {
    return -0.5f * kPi / rc * sinf(kPi * d / rc);
}

// Records whose harmonic rows k_eq_pair_dir stages per round: 64, or 32 for
// orders whose rows would not fit four waves' LDS (nq > 64, order 8).
__device__ __host__ constexpr int pair_dir_chunk(int nq) { return nq > 64 ? 32 : 64; }

// Reverse pass of the angular messages, walked from the neighbour side: the
// wave of atom j holds its mixed state M_j, gathers the centre's
// dE/d(dir_out) once per record and produces the direction-gate adjoints
// dE/dgate[e, G:], their share of dE/dfc, dE/dM_j = sum_e fc tT[e] dHt_i, and
// the injected term's share of dE/dY_e = fc sum_c tI[e, (L, c)] dHt_i[c, :]
// (added to dy; the channel sum goes through a per-wave LDS tile).  Harmonic
// rows of a 64-record chunk are staged in LDS with one parallel load.
template <int LQ, int S>
__global__ void __launch_bounds__(kBlock) k_eq_pair_dir(EqArgs a) {
    constexpr int NQ = LQ * (LQ + 2), LY = NQ + (NQ % 4 == 0 ? 4 : 1);
    using Ln = Lanes<S>;
    constexpr int W = Ln::W;
    constexpr int WT = W + 4;              // T row: channels of one (slot, k), padded
    constexpr int KQ = (NQ + W - 1) / W;   // dE/dY components per lane
    constexpr int RC = pair_dir_chunk(NQ);   // records staged per round
    extern __shared__ float lds[];
    const int j = wave_atom(a.r);
    if (j < 0) return;
    const Ln ln(a.C);
    float *Yc = lds + (threadIdx.x >> 6) * (RC * LY + S * NQ * WT);
    float *T = Yc + RC * LY;
    const int G = a.G, C = a.C, CN = C * NQ, LC = LQ * C, NG = a.NG;
    float MX[NQ], acc[NQ];
    zero(MX);
    zero(acc);
    if (ln.act) load_row(MX, a.mixst + size_t(j) * CN + ln.c * NQ);
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    for (int t0 = tb; t0 < te; t0 += RC) {
        const int cnt = min(RC, te - t0);
        int me = -1, mi = 0;
        float mf = 0.0f, md = 0.0f;
        wave_sync();
        if (ln.lane < cnt) {
            me = a.r.tidx[t0 + ln.lane];
            mi = a.r.tctr[t0 + ln.lane];
            mf = a.tfc[t0 + ln.lane];
            md = a.dfc[me];
            if (mf != 0.0f) {
                float y[NQ];
                load_row(y, a.harm + size_t(me) * NQ);
#pragma unroll
                for (int k = 0; k < NQ; ++k) Yc[ln.lane * LY + k] = y[k];
            }
        }
        wave_sync();
        // every lane loads (clamped indices), so the compiler's waits stay exact
        auto fetch = [&](int q, int &e, float (&dh)[NQ], float (&tt)[LQ], float (&ti)[LQ],
                         float (&yo)[KQ], float &f) {
            const int qq = min(q, cnt - 1);
            const int ec = bcast(me, qq), i = bcast(mi, qq), cl = min(ln.c, C - 1);
            const float fq = bcast(mf, qq);   // every lane joins the shuffle
            f = q < cnt ? fq : 0.0f;
            e = q < cnt ? ec : -1;
#pragma unroll
            for (int u = 0; u < KQ; ++u)
                yo[u] = a.dy_old[(a.dy_old == a.dy ? size_t(ec) * NQ : 0) +
                                 min(ln.c + W * u, NQ - 1)];
            load_row(dh, a.dht + size_t(i) * CN + cl * NQ);
            const float *gr = a.ag + size_t(ec) * NG + G + cl;
#pragma unroll
            for (int L = 0; L < LQ; ++L) {
                tt[L] = gr[L * C];
                ti[L] = gr[LC + L * C];
            }
        };
        // two rounds of gathers in flight
        int e, e1;
        float DH[NQ], tT[LQ], tI[LQ], yo[KQ], fc;
        float DH1[NQ], tT1[LQ], tI1[LQ], yo1[KQ], fc1;
        fetch(ln.slot, e, DH, tT, tI, yo, fc);
        fetch(ln.slot + S, e1, DH1, tT1, tI1, yo1, fc1);
        for (int q0 = 0; q0 < cnt; q0 += S) {
            const int q = q0 + ln.slot;
            int en;
            float DHn[NQ], tTn[LQ], tIn[LQ], yon[KQ], fcn;
            fetch(q + 2 * S, en, DHn, tTn, tIn, yon, fcn);
            const bool on = fc != 0.0f;
            float contrib = 0.0f;
            if (e >= 0 && ln.act) {
                float *dg = a.dgg + size_t(e) * NG + G + ln.c;
                if (on) {
                    float Y[NQ];
                    lds_row<NQ, LY>(Y, Yc, q);
#pragma unroll
                    for (int L = 1; L <= LQ; ++L) {
                        const int st = L * L - 1;
                        float sT = 0.0f, sI = 0.0f;
#pragma unroll
                        for (int m = 0; m < 2 * L + 1; ++m) {
                            sT += DH[st + m] * MX[st + m];
                            sI += DH[st + m] * Y[st + m];
                        }
                        const float t1 = tT[L - 1], t2 = tI[L - 1];
                        dg[(L - 1) * C] = (1.0f - t1 * t1) * fc * sT;
                        dg[LC + (L - 1) * C] = (1.0f - t2 * t2) * fc * sI;
                        contrib += t1 * sT + t2 * sI;
#pragma unroll
                        for (int m = 0; m < 2 * L + 1; ++m) {
                            acc[st + m] += fc * t1 * DH[st + m];
                            T[(ln.slot * NQ + st + m) * WT + ln.c] = fc * t2 * DH[st + m];
                        }
                    }
                } else {
#pragma unroll
                    for (int L = 0; L < LQ; ++L) {
                        dg[L * C] = 0.0f;
                        dg[LC + L * C] = 0.0f;
                    }
                }
            }
            contrib = group_sum(contrib, W);
            const float dold = bcast(md, min(q, kWave - 1));
            if (on && ln.c == 0) a.dfc[e] = dold + contrib;
            wave_sync();
            // the first reverse block writes every record's row (dy holds no
            // earlier shares, so it is not cleared beforehand)
            if (on || (e >= 0 && a.dy_old != a.dy)) {
#pragma unroll
                for (int u = 0; u < KQ; ++u) {
                    const int k = ln.c + W * u;
                    if (k < NQ) {
                        const float *row = T + (ln.slot * NQ + k) * WT;
                        float4 s4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        int c = 0;
                        for (; c + 4 <= C; c += 4) {
                            const float4 t = *reinterpret_cast<const float4 *>(row + c);
                            s4.x += t.x;
                            s4.y += t.y;
                            s4.z += t.z;
                            s4.w += t.w;
                        }
                        float sum = (s4.x + s4.y) + (s4.z + s4.w);
                        for (; c < C; ++c) sum += row[c];
                        a.dy[size_t(e) * NQ + k] = yo[u] + (on ? sum : 0.0f);
                    }
                }
            }
            wave_sync();
            e = e1;
            copy(DH, DH1);
            copy(tT, tT1);
            copy(tI, tI1);
            copy(yo, yo1);
            fc = fc1;
            e1 = en;
            copy(DH1, DHn);
            copy(tT1, tTn);
            copy(tI1, tIn);
            copy(yo1, yon);
            fc1 = fcn;
        }
    }
    fold_slots<S>(acc);
    if (ln.slot == 0 && ln.act) store_row(acc, a.dmix + size_t(j) * CN + ln.c * NQ);
}

// Reverse pass of the scalar messages from the neighbour side: the wave of
// atom j holds V_j (lanes over hidden units), gathers dE/dmsg of the centre
// once per record and produces the group-gate adjoints dE/dgate[e, :G],
// their share of dE/dfc and dE/dV_j = sum_e fc s_e dmsg_i.  Group sums
// P_g = sum_{h in g} dmsg_i[h] V_j[h]: lane reductions when the group width
// is a power of two up to 64 (gmode 0) or a multiple of 64 (gmode 1), else a
// per-wave LDS row (gmode 2).
__global__ void __launch_bounds__(kBlock) k_eq_pair_grp(EqArgs a) {
    extern __shared__ float lds[];
    const int j = wave_atom(a.r);
    if (j < 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int H = a.H, G = a.G, NG = a.NG, gw = H / G, gmode = a.gmode;
    float *T = lds + (threadIdx.x >> 6) * H;
    float Vj[4], vacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = lane + kWave * u;
        Vj[u] = h < H ? a.node[size_t(j) * a.NP + 2 * a.D + h] : 0.0f;
    }
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    for (int t0 = tb; t0 < te; t0 += kWave) {
        const int cnt = min(kWave, te - t0);
        int me = -1, mi = 0;
        float mf = 0.0f, md = 0.0f;
        if (lane < cnt) {
            me = a.r.tidx[t0 + lane];
            mi = a.r.tctr[t0 + lane];
            mf = a.tfc[t0 + lane];
            md = a.dfc[me];
        }
        // every lane loads (clamped indices), so the compiler's waits stay exact
        auto fetch = [&](int q, int &e, float (&dm)[4], float (&sg)[4], float &f) {
            const int qq = min(q, cnt - 1);
            e = lane_get(me, qq);
            const int i = lane_get(mi, qq);
            const float fq = lane_get(mf, qq);
            f = q < cnt ? fq : 0.0f;
            const float *dr = a.dmsg + size_t(i) * H;
            const float *gr = a.ag + size_t(e) * NG;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int h = min(lane + kWave * u, H - 1);
                dm[u] = dr[h];
                sg[u] = gr[h / gw];
            }
        };
        int e, e1;
        float dm[4], sg[4], fc, dm1[4], sg1[4], fc1;
        fetch(0, e, dm, sg, fc);
        fetch(1, e1, dm1, sg1, fc1);
        for (int q = 0; q < cnt; ++q) {
            int en;
            float dmn[4], sgn[4], fcn;
            fetch(q + 2, en, dmn, sgn, fcn);
            const bool on = fc != 0.0f;
            float *dg = a.dgg + size_t(e) * NG;
            float contrib = 0.0f;
            if (on) {
#pragma unroll
                for (int u = 0; u < 4; ++u) vacc[u] += sg[u] * fc * dm[u];
            }
            if (gmode == 0) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (kWave * u < H) {
                        const float P = group_sum(dm[u] * Vj[u], gw);
                        const int h = lane + kWave * u;
                        if (h < H && h % gw == 0) {
                            dg[h / gw] = on ? P * fc * sg[u] * (1.0f - sg[u]) : 0.0f;
                            contrib += P * sg[u];
                        }
                    }
                }
            } else if (gmode == 1) {
                float P = 0.0f;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (kWave * u < H) {
                        P += wave_sum(dm[u] * Vj[u]);
                        if ((kWave * (u + 1)) % gw == 0) {
                            if (lane == 0) {
                                dg[(kWave * u) / gw] = on ? P * fc * sg[u] * (1.0f - sg[u]) : 0.0f;
                                contrib += P * sg[u];
                            }
                            P = 0.0f;
                        }
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int h = lane + kWave * u;
                    if (h < H) T[h] = dm[u] * Vj[u];
                }
                wave_sync();
                for (int g = lane; g < G; g += kWave) {
                    float P = 0.0f;
                    for (int h = g * gw; h < (g + 1) * gw; ++h) P += T[h];
                    const float s = on ? a.ag[size_t(e) * NG + g] : 0.0f;
                    dg[g] = on ? P * fc * s * (1.0f - s) : 0.0f;
                    contrib += P * s;
                }
                wave_sync();
            }
            contrib = wave_sum(contrib);
            const float dold = bcast(md, q);
            if (on && lane == 0) a.dfc[e] = dold + contrib;
            e = e1;
            copy(dm, dm1);
            copy(sg, sg1);
            fc = fc1;
            e1 = en;
            copy(dm1, dmn);
            copy(sg1, sgn);
            fc1 = fcn;
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = lane + kWave * u;
        if (h < H) a.dnode[size_t(j) * a.NP + 2 * a.D + h] = vacc[u];
    }
}

// The same reverse pass with two records in flight per wave: lane c of slot
// s (32 lanes each) owns the CPL contiguous channels c*CPL .. c*CPL+CPL-1 of
// its record, all inside one gate group, so the group's dE/dgate needs only a
// sum over the group's gw / CPL lanes (quad DPP for gw / CPL <= 4) and the
// message rows are read as 16-byte vectors.  Used when H = 32 CPL and CPL
// divides the group width (gmode 3).
template <int CPL>
__global__ void __launch_bounds__(kBlock) k_eq_pair_grp_c(EqArgs a) {
    constexpr int S = 2, SW = kWave / S;
    const int j = wave_atom(a.r);
    if (j < 0) return;
    const int lane = threadIdx.x & (kWave - 1), slot = lane / SW, c = lane % SW;
    const int H = a.H, NG = a.NG, gw = H / a.G, lpg = gw / CPL, g = c / lpg;
    const bool head = c % lpg == 0;
    float Vj[CPL], vacc[CPL];
    {
        const float4 *vr = reinterpret_cast<const float4 *>(a.node + size_t(j) * a.NP + 2 * a.D +
                                                            c * CPL);
#pragma unroll
        for (int u = 0; u < CPL / 4; ++u) {
            const float4 v = vr[u];
            Vj[4 * u] = v.x;
            Vj[4 * u + 1] = v.y;
            Vj[4 * u + 2] = v.z;
            Vj[4 * u + 3] = v.w;
        }
    }
    zero(vacc);
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    for (int t0 = tb; t0 < te; t0 += kWave) {
        const int cnt = min(kWave, te - t0);
        int me = 0, mi = 0;
        float mf = 0.0f, md = 0.0f;
        if (lane < cnt) {
            me = a.r.tidx[t0 + lane];
            mi = a.r.tctr[t0 + lane];
            mf = a.tfc[t0 + lane];
            md = a.dfc[me];
        }
        // every lane loads (clamped indices) and joins the shuffles
        auto fetch = [&](int q, int &e, float (&dm)[CPL], float &sg, float &f) {
            const int qq = min(q, cnt - 1);
            e = bcast(me, qq);
            const int i = bcast(mi, qq);
            const float fq = bcast(mf, qq);
            f = q < cnt ? fq : 0.0f;
            const float4 *dr = reinterpret_cast<const float4 *>(a.dmsg + size_t(i) * H + c * CPL);
#pragma unroll
            for (int u = 0; u < CPL / 4; ++u) {
                const float4 v = dr[u];
                dm[4 * u] = v.x;
                dm[4 * u + 1] = v.y;
                dm[4 * u + 2] = v.z;
                dm[4 * u + 3] = v.w;
            }
            sg = a.ag[size_t(e) * NG + g];
        };
        int e, e1;
        float dm[CPL], dm1[CPL], sg, sg1, fc, fc1;
        fetch(slot, e, dm, sg, fc);
        fetch(slot + S, e1, dm1, sg1, fc1);
        for (int q0 = 0; q0 < cnt; q0 += S) {
            const int q = q0 + slot;
            int en;
            float dmn[CPL], sgn, fcn;
            fetch(q + 2 * S, en, dmn, sgn, fcn);
            const bool on = fc != 0.0f;
            float P = 0.0f;
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                P += dm[u] * Vj[u];
                vacc[u] += on ? sg * fc * dm[u] : 0.0f;
            }
            P = group_sum(P, lpg);
            if (q < cnt && head)
                a.dgg[size_t(e) * NG + g] = on ? P * fc * sg * (1.0f - sg) : 0.0f;
            const float contrib = group_sum(head ? P * sg : 0.0f, SW);
            const float dold = bcast(md, min(q, kWave - 1));
            if (q < cnt && on && c == 0) a.dfc[e] = dold + contrib;
            e = e1;
            copy(dm, dm1);
            sg = sg1;
            fc = fc1;
            e1 = en;
            copy(dm1, dmn);
            sg1 = sgn;
            fc1 = fcn;
        }
    }
    // the two slots' partial sums, added in a fixed order
#pragma unroll
    for (int u = 0; u < CPL; ++u) vacc[u] += __shfl_xor(vacc[u], SW, kWave);
    if (slot == 0) {
        float4 *out = reinterpret_cast<float4 *>(a.dnode + size_t(j) * a.NP + 2 * a.D + c * CPL);
#pragma unroll
        for (int u = 0; u < CPL / 4; ++u)
            out[u] = make_float4(vacc[4 * u], vacc[4 * u + 1], vacc[4 * u + 2], vacc[4 * u + 3]);
    }
}

// Records per matrix-core batch of the edge-MLP reverse kernels.
constexpr int kAdjBatch = 16;

// One lane's share of a batch row: quarter qq of the due row (NTC float4 of
// the column block), 4 MT harmonic values and the old dE/dY values
// qq + 4 i.  Indices are clamped, so every lane loads.
template <int NTC, int NY, int KO>
struct AdjRows {
    float dv[4 * NTC];
    float yv[NY], ov[KO];
};
template <int NTC, int NY, int KO, int NQ>
__device__ __forceinline__ AdjRows<NTC, NY, KO> adj_rows(const float *due, int n4, int qq,
                                                        const float *harm, const float *dy) {
    AdjRows<NTC, NY, KO> st;
    const float4 *src = reinterpret_cast<const float4 *>(due);
#pragma unroll
    for (int i = 0; i < NTC; ++i) {
        const float4 v = src[min(qq * NTC + i, n4 - 1)];
        st.dv[4 * i] = v.x;
        st.dv[4 * i + 1] = v.y;
        st.dv[4 * i + 2] = v.z;
        st.dv[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < NY; ++i) st.yv[i] = harm[min(qq * NY + i, NQ - 1)];
#pragma unroll
    for (int i = 0; i < KO; ++i) st.ov[i] = dy[min(qq + 4 * i, NQ - 1)];
    return st;
}

// Reverse of the factored edge MLP for the records of atom n on one side
// (SIDE 0: the records with centre n, SIDE 1: the records with neighbour n),
// on the matrix cores (v_mfma_f32_16x16x4f32), 16 records at a time.  With
// due = dE/du [rec, d] and Q_n the side's per-atom factor [NQ, d]:
//   dY[rec, k]  += sum_d due[rec, d] Q_n[k, d]
//   dQ_n[k, d]   = sum_rec Y[rec, k] due[rec, d]
// and, from a constant component Y[rec, NQ] = 1, the context adjoint
// dE/dA_n (SIDE 0) or dE/dB_n (SIDE 1) = sum_rec due[rec, :].  A batch's
// due, harmonic and old dE/dY rows are staged in the wave's LDS with one
// lane-parallel load.  The output columns go in blocks of 16 NTC (one block
// for the usual widths); each block walks the records again.
//
// MFMA operand layout: lane l supplies A[l%16][l/16] and B[l/16][l%16]; the
// accumulator register v of lane l holds C[4(l/16) + v][l%16].  For dY the
// k-steps take d = 16 t + 4 (l/16) + s (s = 0..3), so each lane reads its four
// A values with one 16-byte LDS read.
template <int LQ, int NTC, int SIDE>
__global__ void __launch_bounds__(kBlock, 2) k_eq_edge_adj(EqArgs a) {
    constexpr int NQ = LQ * (LQ + 2), MT = (NQ + 16) / 16, KP = 16 * MT;
    constexpr int CW = 16 * NTC, LDU = CW + 4, LDY = KP + 4, LDO = NQ + 1;
    extern __shared__ float lds[];
    const int n = wave_atom(a.r);
    if (n < 0) return;
    const int lane = threadIdx.x & (kWave - 1), g = lane >> 4, r = lane & 15;
    float *dueL = lds + (threadIdx.x >> 6) * a.wlds;   // [16][LDU]
    float *YL = dueL + kAdjBatch * LDU;                 // [16][LDY]
    float *oldL = YL + kAdjBatch * LDY;                 // [16][LDO]
    int *eL = reinterpret_cast<int *>(oldL + kAdjBatch * LDO);
    const int ldd = a.ldd, ldq = 2 * ldd, D = a.D;
    const int b0 = SIDE ? a.r.tptr[n] : a.r.view[4 * n];
    const int b1 = SIDE ? a.r.tptr[n + 1] : a.r.view[4 * n + 1];
    float *dyo = a.dy;
    const float *Qn = a.qbuf + size_t(n) * NQ * ldq + SIDE * ldd;
    float *dQo = a.dqbuf + size_t(n) * NQ * ldq + SIDE * ldd;
    for (int c0 = 0; c0 < ldd; c0 += CW) {
        const int ntv = min(NTC, (ldd - c0) / 16);   // n-tiles of this column block
        floatx4 Bq[NTC][MT];
#pragma unroll
        for (int t = 0; t < NTC; ++t)
#pragma unroll
            for (int nt = 0; nt < MT; ++nt) {
                const int k = 16 * nt + r;
                const float4 v = *reinterpret_cast<const float4 *>(
                    Qn + size_t(min(k, NQ - 1)) * ldq + c0 + 16 * min(t, ntv - 1) + 4 * g);
                const bool ok = k < NQ && t < ntv;
                Bq[t][nt] = floatx4{ok ? v.x : 0.0f, ok ? v.y : 0.0f, ok ? v.z : 0.0f,
                                    ok ? v.w : 0.0f};
            }
        floatx4 acc[MT][NTC];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NTC; ++nt) acc[mt][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        // The rows of batch b + 1 are loaded into registers while batch b is
        // on the matrix cores, and written to LDS once its reads are done;
        // the record ids run one batch further ahead.  Lane l stages row
        // l / 4 of a batch, quarter l % 4 of each row.
        const int rec = lane >> 2, qq = lane & 3;
        constexpr int KO = (NQ + 3) / 4;
        auto record_of = [&](int t0) {
            const int rv = min(rec, max(min(kAdjBatch, b1 - t0), 1) - 1);
            return SIDE ? a.r.tidx[min(t0 + rv, b1 - 1)] : min(t0 + rv, b1 - 1);
        };
        AdjRows<NTC, 4 * MT, KO> st;
        int e_cur = 0, e_nxt = 0;
        if (b1 > b0) {
            e_cur = record_of(b0);
            e_nxt = record_of(b0 + kAdjBatch);
            st = adj_rows<NTC, 4 * MT, KO, NQ>(a.due + size_t(e_cur) * ldd + c0, 4 * ntv, qq,
                                               a.harm + size_t(e_cur) * NQ,
                                               dyo + size_t(e_cur) * NQ);
        }
        for (int t0 = b0; t0 < b1; t0 += kAdjBatch) {
            const int cnt = min(kAdjBatch, b1 - t0);
            wave_sync();
            {
                const bool live = rec < cnt;
#pragma unroll
                for (int i = 0; i < NTC; ++i)
                    *reinterpret_cast<float4 *>(dueL + rec * LDU + 4 * (qq * NTC + i)) =
                        make_float4(st.dv[4 * i], st.dv[4 * i + 1], st.dv[4 * i + 2],
                                    st.dv[4 * i + 3]);
#pragma unroll
                for (int i = 0; i < 4 * MT; ++i) {
                    const int k = 4 * qq * MT + i;
                    const float y = k < NQ ? st.yv[i] : (k == NQ ? 1.0f : 0.0f);
                    YL[rec * LDY + k] = live ? y : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < KO; ++i)
                    if (qq + 4 * i < NQ) oldL[rec * LDO + qq + 4 * i] = st.ov[i];
                if (qq == 0) eL[rec] = e_cur;
            }
            wave_sync();
            if (t0 + kAdjBatch < b1) {
                e_cur = e_nxt;
                e_nxt = record_of(t0 + 2 * kAdjBatch);
                st = adj_rows<NTC, 4 * MT, KO, NQ>(a.due + size_t(e_cur) * ldd + c0, 4 * ntv, qq,
                                                   a.harm + size_t(e_cur) * NQ,
                                                   dyo + size_t(e_cur) * NQ);
            }
            // two independent accumulation chains per tile
            floatx4 pc[2][MT];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int nt = 0; nt < MT; ++nt) pc[h][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < NTC; ++t) {
                const float4 av = *reinterpret_cast<const float4 *>(dueL + r * LDU + 16 * t + 4 * g);
#pragma unroll
                for (int nt = 0; nt < MT; ++nt) {
                    pc[0][nt] = mfma4(av.x, Bq[t][nt][0], pc[0][nt]);
                    pc[1][nt] = mfma4(av.y, Bq[t][nt][1], pc[1][nt]);
                    pc[0][nt] = mfma4(av.z, Bq[t][nt][2], pc[0][nt]);
                    pc[1][nt] = mfma4(av.w, Bq[t][nt][3], pc[1][nt]);
                }
            }
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int rr = 4 * s4 + g;
                float ya[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) ya[mt] = YL[rr * LDY + 16 * mt + r];
#pragma unroll
                for (int nt = 0; nt < NTC; ++nt) {
                    const float b = dueL[rr * LDU + 16 * nt + r];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma4(ya[mt], b, acc[mt][nt]);
                }
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int rr = 4 * g + v;
                if (rr < cnt) {
                    const size_t row = size_t(eL[rr]) * NQ;
#pragma unroll
                    for (int nt = 0; nt < MT; ++nt) {
                        const int k = 16 * nt + r;
                        if (k < NQ) dyo[row + k] = oldL[rr * LDO + k] + (pc[0][nt][v] + pc[1][nt][v]);
                    }
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NTC; ++nt) {
                if (nt < ntv) {
                    const int d = c0 + 16 * nt + r;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int k = 16 * mt + 4 * g + v;
                        if (k < NQ)
                            dQo[size_t(k) * ldq + d] = acc[mt][nt][v];
                        else if (k == NQ && d < D)
                            a.dnode[size_t(n) * a.NP + SIDE * D + d] = acc[mt][nt][v];
                    }
                }
            }
    }
}

// dst[t] = src[idx[t]] for t < E; also clears z0[0, E) and z1[0, n1).
__global__ void k_gather_f(int64_t E, const int32_t *idx, const float *src, float *dst,
                           float *z0, float *z1, int n1) {
    int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t < E) {
        dst[t] = src[idx[t]];
        z0[t] = 0.0f;
    }
    if (t < n1) z1[t] = 0.0f;
}

// Reverse of the direction encoder: dE/ds[i, n, k] = scale[k] sum_c
// enc[(L(k)-1) C + c][n] dE/dout[i, c, k] (zero for k >= nq).  Same layout as
// k_eq_encode.
__global__ void __launch_bounds__(256) k_eq_encoder_backward(int N, const float *ddir0,
                                                            const float *enc,
                                                            const float *scale, int lq, int C,
                                                            int nq, int na, int nlm, int wrow,
                                                            float *dmom) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
    float *W = lds;                                  // [lq C][na]
    float *row = lds + lq * C * na + wave * wrow;    // [C][nq]
    for (int o = threadIdx.x; o < lq * C * na; o += blockDim.x) W[o] = enc[o];
    __syncthreads();
    for (int i0 = blockIdx.x * 4; i0 < N; i0 += gridDim.x * 4) {
        const int i = i0 + wave;
        if (i >= N) continue;
        wave_sync();
        stage_row(row, ddir0 + size_t(i) * C * nq, C * nq);
        wave_sync();
        for (int o = lane; o < na * nlm; o += kWave) {
            const int n = o / nlm, k = o - n * nlm;
            float g = 0.0f;
            if (k < nq) {
                const int L = order_of(k);
                for (int c = 0; c < C; ++c) g += W[((L - 1) * C + c) * na + n] * row[c * nq + k];
                g *= scale[k];
            }
            dmom[size_t(i) * na * nlm + o] = g;
        }
    }
}

// dE/du of the harmonics: sum_k dY_k scale_k db_k/du, added to dv.xyz; dv.w
// gains dE/dfc fc'(d) and the radial-basis term sum_k dE/drb_k drb_k/dd.
template <int LQ>
__global__ void k_eq_harmonic_backward(int64_t E, Records r, const float *fcv, const float *dy,
                                       const float *dfc, const float *drb,
                                       const float *rbd, int ldrb, int kb, float cutoff,
                                       const float *ztab, EdgeZ zoff, const float *scale,
                                       float4 *dv) {
    constexpr int NQ = LQ * (LQ + 2);
    int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    int i = r.ctr[e];
    if (!(e >= r.view[4 * i] && e < r.view[4 * i + 1])) return;
    float gs[NQ];
    load_row(gs, dy + size_t(e) * NQ);
    float4 v = r.vec[e];
    float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
    float x = v.x * inv, y = v.y * inv, z = v.z * inv;
    float zp[LQ + 1], wr[LQ + 1], wi[LQ + 1];
    zp[0] = 1.0f;
    wr[0] = 1.0f;
    wi[0] = 0.0f;
#pragma unroll
    for (int k = 1; k <= LQ; ++k) {
        zp[k] = zp[k - 1] * z;
        wr[k] = wr[k - 1] * x - wi[k - 1] * y;
        wi[k] = wr[k - 1] * y + wi[k - 1] * x;
    }
    float dx = 0.0f, dyy = 0.0f, dz = 0.0f;
    int idx = 0;
#pragma unroll
    for (int L = 1; L <= LQ; ++L) {
#pragma unroll
        for (int n1 = 0; n1 <= L; ++n1) {
            const float *Z = ztab + zoff.off[L] + n1 * (L + 1);
            float zf = 0.0f, zfp = 0.0f;
#pragma unroll
            for (int q = ((L + n1) & 1); q <= L - n1; q += 2) {
                zf += Z[q] * zp[q];
                if (q > 0) zfp += float(q) * Z[q] * zp[q - 1];
            }
#pragma unroll
            for (int part = 0; part < (n1 == 0 ? 1 : 2); ++part, ++idx) {
                float w = gs[idx] * scale[idx];
                if (n1 == 0) {
                    dz += w * zfp;
                } else if (part == 0) {
                    dx += w * zf * float(n1) * wr[n1 - 1];
                    dyy -= w * zf * float(n1) * wi[n1 - 1];
                    dz += w * zfp * wr[n1];
                } else {
                    dx += w * zf * float(n1) * wi[n1 - 1];
                    dyy += w * zf * float(n1) * wr[n1 - 1];
                    dz += w * zfp * wi[n1];
                }
            }
        }
    }
    float4 acc = dv[e];
    acc.x += dx;
    acc.y += dyy;
    acc.z += dz;
    if (fcv[e] != 0.0f) {
        // 16-byte row reads (ldrb is a multiple of 4); the padding columns
        // are skipped, so the sum is the plain k-ordered one
        const float4 *d4 = reinterpret_cast<const float4 *>(drb + size_t(e) * ldrb);
        const float4 *r4 = reinterpret_cast<const float4 *>(rbd + size_t(e) * ldrb);
        float t = 0.0f;
        for (int q = 0; 4 * q < kb; ++q) {
            const float4 a = d4[q], b = r4[q];
            const int k = 4 * q;
            t += a.x * b.x;
            if (k + 1 < kb) t += a.y * b.y;
            if (k + 2 < kb) t += a.z * b.z;
            if (k + 3 < kb) t += a.w * b.w;
        }
        acc.w += dfc[e] * cutoff_slope(v.w, cutoff) + t;
    }
    dv[e] = acc;
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static void expect(ModelImpl &m, const std::string &name, int64_t n) { m.expected[name] = n; }

// Records per wave in the angular-state loops: slots of 64 / S lanes hold
// one channel per lane.
static int eq_slots(int C) { return C > 32 ? 1 : C > 16 ? 2 : 4; }

// Launches kernel template k<LQ> for the runtime order lq (1..8).
#define EQ_LAUNCH(k, lq, grid, block, lds, s, ...)                                         \
    do {                                                                                  \
        switch (lq) {                                                                     \
        case 1: hipLaunchKernelGGL(k<1>, grid, block, lds, s, __VA_ARGS__); break;        \
        case 2: hipLaunchKernelGGL(k<2>, grid, block, lds, s, __VA_ARGS__); break;        \
        case 3: hipLaunchKernelGGL(k<3>, grid, block, lds, s, __VA_ARGS__); break;        \
        case 4: hipLaunchKernelGGL(k<4>, grid, block, lds, s, __VA_ARGS__); break;        \
        case 5: hipLaunchKernelGGL(k<5>, grid, block, lds, s, __VA_ARGS__); break;        \
        case 6: hipLaunchKernelGGL(k<6>, grid, block, lds, s, __VA_ARGS__); break;        \
        case 7: hipLaunchKernelGGL(k<7>, grid, block, lds, s, __VA_ARGS__); break;        \
        default: hipLaunchKernelGGL(k<8>, grid, block, lds, s, __VA_ARGS__); break;       \
        }                                                                                 \
        RUNE_HIP_CHECK(hipGetLastError());                                                \
    } while (0)

#define EQ_CASE_S(k, L, S, grid, block, lds, s, ...)                                      \
    case S:                                                                               \
        if ((lds) > 65536)                                                                \
            RUNE_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&k<L, S>), \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, \
                                               int(lds)));                                \
        hipLaunchKernelGGL((k<L, S>), grid, block, lds, s, __VA_ARGS__);                  \
        break;
#define EQ_CASE_L(k, L, S, ...)                                                           \
    case L:                                                                               \
        switch (S) {                                                                      \
        EQ_CASE_S(k, L, 1, __VA_ARGS__)                                                   \
        EQ_CASE_S(k, L, 2, __VA_ARGS__)                                                   \
        default:                                                                          \
        switch (4) { EQ_CASE_S(k, L, 4, __VA_ARGS__) }                                    \
        break;                                                                            \
        }                                                                                 \
        break;
// Launches kernel template k<LQ, S> of the per-atom record loops.
#define EQ_LAUNCH_S(k, lq, S, ...)                                                         \
    do {                                                                                  \
        switch (lq) {                                                                     \
        EQ_CASE_L(k, 1, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 2, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 3, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 4, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 5, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 6, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 7, S, __VA_ARGS__)                                                   \
        EQ_CASE_L(k, 8, S, __VA_ARGS__)                                                   \
        }                                                                                 \
        RUNE_HIP_CHECK(hipGetLastError());                                                \
    } while (0)

// Output columns per lane of the edge-MLP kernels: up to 4 (64 each), fewer
// when the per-atom factor and the radial-basis weights would not fit in
// about 140 registers.
static int edge_dmc(int lq, int D) {
    const int nq = lq * (lq + 2);
    int c = std::min(ceil_div(D, kWave), 4);
    while (c > 1 && (nq + kRbRegs) * c > 140) --c;
    return c;
}

// Row stride of the per-record [E, D] arrays: whole column blocks of the
// edge-MLP kernels.
static int edge_ld(int lq, int D) {
    const int dmc = edge_dmc(lq, D);
    return ceil_div(D, kWave * dmc) * kWave * dmc;
}

// Output column tiles per block of the edge-MLP reverse kernels: 16 x 4, 8
// or 12 columns, as many as the register budget allows for the order lq.
static int adj_ntc(int lq, int ldd) {
    const int nq = lq * (lq + 2), mt = (nq + 16) / 16, nt = ldd / 16;
    const int cap = mt <= 2 ? 6 : mt == 3 ? 6 : 4;
    const int want = nt <= 4 ? 4 : 6;
    return std::min(cap, want);
}

#define EQ_CASE_A(k, L, T, S, ...)                                                        \
    case T: hipLaunchKernelGGL((k<L, T, S>), __VA_ARGS__); break;
#define EQ_CASE_AL(k, L, ntc, S, ...)                                                     \
    case L:                                                                               \
        switch (ntc) {                                                                    \
        EQ_CASE_A(k, L, 6, S, __VA_ARGS__)                                                \
        default: hipLaunchKernelGGL((k<L, 4, S>), __VA_ARGS__); break;                    \
        }                                                                                 \
        break;
// Launches kernel template k<LQ, NTC, S> (the pairs adj_ntc can choose).
#define EQ_LAUNCH_A(k, lq, ntc, S, ...)                                                    \
    do {                                                                                  \
        switch (lq) {                                                                     \
        EQ_CASE_AL(k, 1, ntc, S, __VA_ARGS__)                                             \
        EQ_CASE_AL(k, 2, ntc, S, __VA_ARGS__)                                             \
        EQ_CASE_AL(k, 3, ntc, S, __VA_ARGS__)                                             \
        EQ_CASE_AL(k, 4, ntc, S, __VA_ARGS__)                                             \
        case 5:                                                                           \
            if (ntc == 6)                                                                 \
                hipLaunchKernelGGL((k<5, 6, S>), __VA_ARGS__);                            \
            else                                                                          \
                hipLaunchKernelGGL((k<5, 4, S>), __VA_ARGS__);                            \
            break;                                                                        \
        case 6: hipLaunchKernelGGL((k<6, 4, S>), __VA_ARGS__); break;                     \
        case 7: hipLaunchKernelGGL((k<7, 4, S>), __VA_ARGS__); break;                     \
        default: hipLaunchKernelGGL((k<8, 4, S>), __VA_ARGS__); break;                    \
        }                                                                                 \
        RUNE_HIP_CHECK(hipGetLastError());                                                \
    } while (0)

#define EQ_CASE_D(k, L, D, grid, block, lds, s, ...)                                      \
    case D:                                                                               \
        if ((lds) > 65536)                                                                \
            RUNE_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&k<L, D>), \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, \
                                               int(lds)));                                \
        hipLaunchKernelGGL((k<L, D>), grid, block, lds, s, __VA_ARGS__);                  \
        break;
#define EQ_CASE_L4(k, L, dmc, ...)                                                        \
    case L:                                                                               \
        switch (dmc) {                                                                    \
        EQ_CASE_D(k, L, 4, __VA_ARGS__)                                                   \
        EQ_CASE_D(k, L, 3, __VA_ARGS__)                                                   \
        EQ_CASE_D(k, L, 2, __VA_ARGS__)                                                   \
        default: EQ_CASE_D(k, L, 1, __VA_ARGS__)                                          \
        }                                                                                 \
        break;
#define EQ_CASE_L3(k, L, dmc, ...)                                                        \
    case L:                                                                               \
        switch (dmc) {                                                                    \
        EQ_CASE_D(k, L, 3, __VA_ARGS__)                                                   \
        EQ_CASE_D(k, L, 2, __VA_ARGS__)                                                   \
        default: EQ_CASE_D(k, L, 1, __VA_ARGS__)                                          \
        }                                                                                 \
        break;
#define EQ_CASE_L2(k, L, dmc, ...)                                                        \
    case L:                                                                               \
        switch (dmc) {                                                                    \
        EQ_CASE_D(k, L, 2, __VA_ARGS__)                                                   \
        default: EQ_CASE_D(k, L, 1, __VA_ARGS__)                                          \
        }                                                                                 \
        break;
// Launches kernel template k<LQ, DMC> (the pairs edge_dmc can choose).
#define EQ_LAUNCH_D(k, lq, dmc, ...)                                                       \
    do {                                                                                  \
        switch (lq) {                                                                     \
        EQ_CASE_L4(k, 1, dmc, __VA_ARGS__)                                                \
        EQ_CASE_L4(k, 2, dmc, __VA_ARGS__)                                                \
        EQ_CASE_L4(k, 3, dmc, __VA_ARGS__)                                                \
        EQ_CASE_L3(k, 4, dmc, __VA_ARGS__)                                                \
        EQ_CASE_L2(k, 5, dmc, __VA_ARGS__)                                                \
        EQ_CASE_L2(k, 6, dmc, __VA_ARGS__)                                                \
        default:                                                                          \
            if (lq == 7) {                                                                \
                switch (1) { EQ_CASE_D(k, 7, 1, __VA_ARGS__) }                            \
            } else {                                                                      \
                switch (1) { EQ_CASE_D(k, 8, 1, __VA_ARGS__) }                            \
            }                                                                             \
            break;                                                                        \
        }                                                                                 \
        RUNE_HIP_CHECK(hipGetLastError());                                                \
    } while (0)

// Channel mixing per order (k_eq_mix).
template <int LQ>
static void launch_mix_lq(int C, int N, const float *w, const float *in, int trans,
                          const float *add, const float *add_t, float *out, hipStream_t s) {
    constexpr int NQ = LQ * (LQ + 2);
    const int grid = std::max(1, std::min(ceil_div(N, 4), 4096));
    const int mt = ceil_div(C, 16), cp = 16 * mt;
    const size_t lds = sizeof(float) * (8 * ((size_t(C) * NQ + 3) & ~size_t(3)) +
                                        (mt > 2 ? size_t(LQ) * cp * cp : 0));
    switch (mt) {
    case 1: hipLaunchKernelGGL((k_eq_mix<LQ, 1>), dim3(grid), dim3(256), lds, s, N, w, in, C, trans, add, add_t, out); break;
    case 2: hipLaunchKernelGGL((k_eq_mix<LQ, 2>), dim3(grid), dim3(256), lds, s, N, w, in, C, trans, add, add_t, out); break;
    case 3: hipLaunchKernelGGL((k_eq_mix<LQ, 3>), dim3(grid), dim3(256), lds, s, N, w, in, C, trans, add, add_t, out); break;
    default:
        if (lds > 65536)
            RUNE_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_eq_mix<LQ, 4>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               int(lds)));
        hipLaunchKernelGGL((k_eq_mix<LQ, 4>), dim3(grid), dim3(256), lds, s, N, w, in, C, trans, add, add_t, out);
        break;
    }
    RUNE_HIP_CHECK(hipGetLastError());
}

static void launch_mix(int lq, int C, int N, const float *w, const float *in, int trans,
                       const float *add, const float *add_t, float *out, hipStream_t s) {
    if (N == 0) return;
    switch (lq) {
    case 1: launch_mix_lq<1>(C, N, w, in, trans, add, add_t, out, s); break;
    case 2: launch_mix_lq<2>(C, N, w, in, trans, add, add_t, out, s); break;
    case 3: launch_mix_lq<3>(C, N, w, in, trans, add, add_t, out, s); break;
    case 4: launch_mix_lq<4>(C, N, w, in, trans, add, add_t, out, s); break;
    case 5: launch_mix_lq<5>(C, N, w, in, trans, add, add_t, out, s); break;
    case 6: launch_mix_lq<6>(C, N, w, in, trans, add, add_t, out, s); break;
    case 7: launch_mix_lq<7>(C, N, w, in, trans, add, add_t, out, s); break;
    default: launch_mix_lq<8>(C, N, w, in, trans, add, add_t, out, s); break;
    }
}

void validate_equivariant(ModelImpl &m) {
    const rune_model_config &c = m.cfg;
    const int lq = c.equivariant_l_max, C = c.equivariant_channels;
    RUNE_REQUIRE(lq >= 1 && lq <= std::min(c.l_max, kMaxL), RUNE_ERR_ARGUMENT,
                 "equivariant_l_max must be in 1..min(l_max, 8)");
    RUNE_REQUIRE(C >= 1 && C <= kWave, RUNE_ERR_ARGUMENT,
                 "equivariant blocks support equivariant_channels in 1..64");
    RUNE_REQUIRE(c.message_groups >= 1 && c.message_groups <= kWave, RUNE_ERR_ARGUMENT,
                 "message_groups must be in 1..64");
    RUNE_REQUIRE(c.hidden_dim <= 4 * kWave, RUNE_ERR_ARGUMENT,
                 "equivariant blocks support hidden_dim <= 256");
    RUNE_REQUIRE(c.message_dim <= 4 * kWave, RUNE_ERR_ARGUMENT,
                 "equivariant blocks support message_dim <= 256");
    RUNE_REQUIRE(c.hidden_dim % c.message_groups == 0, RUNE_ERR_ARGUMENT,
                 "hidden_dim must be divisible by message_groups");
}

void define_expected_equivariant(ModelImpl &m) {
    const rune_model_config &c = m.cfg;
    const int64_t T = c.n_types, H = c.hidden_dim, D = c.message_dim, P = c.pair_dim;
    const int64_t G = c.message_groups, kb = c.message_basis_size;
    const int64_t lq = c.equivariant_l_max, C = c.equivariant_channels, W = lq * C;
    for (int L = 0; L < lq; ++L)
        expect(m, "direction_encoder.projections." + std::to_string(L) + ".weight",
               C * c.n_desc_angular);
    for (int b = 0; b < c.message_layers; ++b) {
        std::string p = "message_blocks." + std::to_string(b) + ".";
        expect(m, p + "input_norm.weight", H);
        expect(m, p + "center_context.weight", D * H);
        expect(m, p + "neighbor_context.weight", D * H);
        expect(m, p + "pair_embedding.weight", T * T * P);
        expect(m, p + "edge_mlp.0.weight", D * (kb + P + 2 * D + 2 * W));
        expect(m, p + "edge_mlp.0.bias", D);
        expect(m, p + "group_gate.weight", G * D);
        expect(m, p + "group_gate.bias", G);
        expect(m, p + "direction_gates.weight", 2 * W * D);
        expect(m, p + "direction_gates.bias", 2 * W);
        expect(m, p + "value_projection.weight", H * H);
        for (int L = 0; L < lq; ++L)
            expect(m, p + "direction_mix." + std::to_string(L) + ".weight", C * C);
        expect(m, p + "message_norm.weight", H);
        expect(m, p + "update.0.weight", D * (H + W));
        expect(m, p + "update.0.bias", D);
        expect(m, p + "update.2.weight", H * D);
        expect(m, p + "update.2.bias", H);
    }
}

// A = W[:, c0:c0+D] @ ctx   ([D, D] x [D, H] -> [D, H]), double accumulation
static std::vector<float> compose(const std::vector<float> &w, int rows, int K, int c0,
                                  const std::vector<float> &ctx, int D, int H) {
    std::vector<float> out(size_t(rows) * H);
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < H; ++h) {
            double acc = 0.0;
            for (int d = 0; d < D; ++d)
                acc += double(w[size_t(r) * K + c0 + d]) * double(ctx[size_t(d) * H + h]);
            out[size_t(r) * H + h] = float(acc);
        }
    return out;
}

void pack_equivariant(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off) {
    const rune_model_config &c = m.cfg;
    const int T = c.n_types, H = c.hidden_dim, D = c.message_dim, P = c.pair_dim;
    const int G = c.message_groups, kb = c.message_basis_size;
    const int lq = c.equivariant_l_max, C = c.equivariant_channels, W = lq * C;
    const int K = kb + P + 2 * D + 2 * W, NP = 2 * D + H, NG = G + 2 * W;
    std::vector<float> enc;
    for (int L = 0; L < lq; ++L) {
        const auto &t = m.tensor("direction_encoder.projections." + std::to_string(L) + ".weight");
        enc.insert(enc.end(), t.begin(), t.end());
    }
    off["eq_enc"] = pk.put(enc);
    // orthonormal scale sqrt(2 C3B), halved inside the root at m = 0 (descriptor.py:626-637)
    const auto &c3b = m.tensor("descriptor.angular.C3B");
    const int nq = lq * (lq + 2);
    std::vector<float> scale(nq);
    for (int k = 0; k < nq; ++k) {
        float v = c3b[k] * 2.0f;
        int L = 1;
        while ((L + 1) * (L + 1) - 1 <= k) ++L;
        if (k == L * L - 1) v *= 0.5f;
        scale[k] = std::sqrt(v);
    }
    off["eq_scale"] = pk.put(scale);
    for (int b = 0; b < c.message_layers; ++b) {
        std::string p = "message_blocks." + std::to_string(b) + ".";
        const auto &we = m.tensor(p + "edge_mlp.0.weight");     // [D, K]
        const auto &win = m.tensor(p + "input_norm.weight");
        std::vector<float> node = compose(we, D, K, kb + P, m.tensor(p + "center_context.weight"),
                                          D, H);
        std::vector<float> nb = compose(we, D, K, kb + P + D,
                                        m.tensor(p + "neighbor_context.weight"), D, H);
        node.insert(node.end(), nb.begin(), nb.end());
        const auto &wv = m.tensor(p + "value_projection.weight");
        node.insert(node.end(), wv.begin(), wv.end());
        node = fold_cols(node, NP, H, win.data());
        off[p + "node_f"] = pk.put(node);
        off[p + "node_fT"] = pk.put(transpose(node, NP, H));
        std::vector<float> wx = columns(we, D, K, 0, kb);                    // [D, kb]
        std::vector<float> wp = columns(we, D, K, kb + P + 2 * D, K);        // [D, 2W]
        // factored edge MLP: [kb, D] radial-basis rows and [lq C, D] probe rows,
        // the neighbour probes signed (-1)^L
        off[p + "edge_rbT"] = pk.put(transpose(wx, D, kb));
        std::vector<float> pc(size_t(W) * D), pn(size_t(W) * D);
        for (int L = 1; L <= lq; ++L)
            for (int cc = 0; cc < C; ++cc) {
                const int row = (L - 1) * C + cc;
                const float sg = (L & 1) ? -1.0f : 1.0f;
                for (int r = 0; r < D; ++r) {
                    pc[size_t(row) * D + r] = wp[size_t(r) * 2 * W + row];
                    pn[size_t(row) * D + r] = sg * wp[size_t(r) * 2 * W + W + row];
                }
            }
        off[p + "probe_c"] = pk.put(pc);
        off[p + "probe_n"] = pk.put(pn);
        const int ldd = edge_ld(lq, D);
        std::vector<float> cat(size_t(W) * 2 * ldd, 0.0f);
        for (int row = 0; row < W; ++row)
            for (int r = 0; r < D; ++r) {
                cat[size_t(row) * 2 * ldd + r] = pc[size_t(row) * D + r];
                cat[size_t(row) * 2 * ldd + ldd + r] = pn[size_t(row) * D + r];
            }
        off[p + "probe_cat"] = pk.put(cat);
        off[p + "pair_proj"] = pk.put(pair_projection(m.tensor(p + "pair_embedding.weight"), we,
                                                      m.tensor(p + "edge_mlp.0.bias"), T * T, P,
                                                      D, K, kb));
        std::vector<float> gate = m.tensor(p + "group_gate.weight");
        const auto &dg = m.tensor(p + "direction_gates.weight");
        gate.insert(gate.end(), dg.begin(), dg.end());
        std::vector<float> gb = m.tensor(p + "group_gate.bias");
        const auto &db = m.tensor(p + "direction_gates.bias");
        gb.insert(gb.end(), db.begin(), db.end());
        off[p + "gate"] = pk.put(gate);
        off[p + "gate_T"] = pk.put(transpose(gate, NG, D));
        {
            std::vector<float> gtp = transpose(gate, NG, D);
            gtp.resize(size_t(edge_ld(lq, D)) * NG, 0.0f);
            off[p + "gate_Tp"] = pk.put(gtp);
        }
        off[p + "gate_b"] = pk.put(gb);
        std::vector<float> mix;
        for (int L = 0; L < lq; ++L) {
            const auto &t = m.tensor(p + "direction_mix." + std::to_string(L) + ".weight");
            mix.insert(mix.end(), t.begin(), t.end());
        }
        off[p + "mix"] = pk.put(mix);
        std::vector<float> wmsg = m.tensor(p + "message_norm.weight");
        wmsg.resize(H + W, 1.0f);
        std::vector<float> up1 = fold_cols(m.tensor(p + "update.0.weight"), D, H + W, wmsg.data());
        off[p + "up1_f"] = pk.put(up1);
        off[p + "up1_fT"] = pk.put(transpose(up1, D, H + W));
        off[p + "up1_b"] = pk.put(m.tensor(p + "update.0.bias"));
        const auto &up2 = m.tensor(p + "update.2.weight");
        off[p + "up2"] = pk.put(up2);
        off[p + "up2_T"] = pk.put(transpose(up2, H, D));
        off[p + "up2_b"] = pk.put(m.tensor(p + "update.2.bias"));
    }
}

void bind_equivariant(ModelImpl &m, const PackedLookup &P) {
    const rune_model_config &c = m.cfg;
    const int W = c.equivariant_l_max * c.equivariant_channels;
    m.enc_w = P("eq_enc");
    m.harm_scale = P("eq_scale");
    m.msg.resize(c.message_layers);
    for (int b = 0; b < c.message_layers; ++b) {
        std::string p = "message_blocks." + std::to_string(b) + ".";
        MessageWeights &w = m.msg[b];
        w.NP = 2 * c.message_dim + c.hidden_dim;
        w.NG = c.message_groups + 2 * W;
        w.KX = c.message_basis_size + 2 * W;
        w.ld_edge_x = (w.KX + 3) & ~3;
        w.node_f = P(p + "node_f");
        w.node_fT = P(p + "node_fT");
        w.edge_rbT = P(p + "edge_rbT");
        w.probe_c = P(p + "probe_c");
        w.probe_n = P(p + "probe_n");
        w.probe_cat = P(p + "probe_cat");
        w.gate_Tp = P(p + "gate_Tp");
        w.pair_proj = P(p + "pair_proj");
        w.gate = P(p + "gate");
        w.gate_T = P(p + "gate_T");
        w.gate_b = P(p + "gate_b");
        w.mix = P(p + "mix");
        w.up1_f = P(p + "up1_f");
        w.up1_fT = P(p + "up1_fT");
        w.up1_b = P(p + "up1_b");
        w.up2 = P(p + "up2");
        w.up2_T = P(p + "up2_T");
        w.up2_b = P(p + "up2_b");
    }
}

MessagePlan plan_equivariant(ModelImpl &m, Arena &ar, int N, int64_t E) {
    MessagePlan p;
    const rune_model_config &c = m.cfg;
    const size_t n = size_t(N), e = size_t(std::max<int64_t>(E, 1));
    const int H = c.hidden_dim, D = c.message_dim, lq = c.equivariant_l_max;
    const int C = c.equivariant_channels, W = lq * C, nq = lq * (lq + 2), CN = C * nq;
    const int NP = 2 * D + H, NG = c.message_groups + 2 * W;
    p.N = N;
    p.E = E;
    p.ldrb = (c.message_basis_size + 3) & ~3;
    p.o_gd = ar.add(16 * e);
    p.o_dmom = ar.add(4 * n * m.desc.na * m.desc.nlm);
    p.i_rb = p.add(ar, 4 * e * p.ldrb);
    p.i_fc = p.add(ar, 4 * e);
    p.i_tfc = p.add(ar, 4 * e);
    p.i_pair = p.add(ar, 4 * e);
    p.i_dv = p.add(ar, 16 * e);
    p.i_harm = p.add(ar, 4 * e * nq);
    p.i_dharm = p.add(ar, 4 * e * nq);
    p.i_zero = p.add(ar, 4 * 128);   // a zero row of >= nq floats
    p.i_dfc = p.add(ar, 4 * e);
    p.i_drb = p.add(ar, 4 * e * p.ldrb);
    p.i_rbd = p.add(ar, 4 * e * p.ldrb);
    int dir0 = p.add(ar, 4 * n * CN);
    p.ld_edge = edge_ld(lq, D);
    const size_t ldd = size_t(p.ld_edge);
    int eh = p.add(ar, 4 * e * ldd);       // shared by the blocks (forward only)
    for (int b = 0; b < c.message_layers; ++b) {
        BlockBuffers bb;
        bb.h_out = p.add(ar, 4 * n * H);
        bb.rin = p.add(ar, 4 * n);
        bb.vs = p.add(ar, 4 * n * NP);
        bb.ue = p.add(ar, 4 * e * ldd);
        bb.eh = eh;
        bb.gv = p.add(ar, 4 * e * NG);
        bb.msg = p.add(ar, 4 * n * H);
        bb.rm = p.add(ar, 4 * n);
        bb.uin = p.add(ar, 4 * n * (H + W));
        bb.u1 = p.add(ar, 4 * n * D);
        bb.z1 = p.add(ar, 4 * n * D);
        bb.dir_in = b == 0 ? dir0 : p.blocks[b - 1].dir_out;
        bb.dir_out = p.add(ar, 4 * n * CN);
        bb.mixstate = p.add(ar, 4 * n * CN);
        bb.q = p.add(ar, 4 * n * nq * 2 * ldd);
        p.blocks.push_back(bb);
    }
    p.t_dz1 = p.add(ar, 4 * n * D);
    p.t_duin = p.add(ar, 4 * n * (H + W));
    p.t_dmsg = p.add(ar, 4 * n * H);
    p.t_dvsum = p.add(ar, 4 * n * CN);     // dE/d(dir_out) total
    p.t_dgv = p.add(ar, 4 * e * NG);
    p.t_due = p.add(ar, 4 * e * ldd);
    p.t_dq = p.add(ar, 4 * n * nq * 2 * ldd);
    p.t_dhk = p.add(ar, 4 * n * CN);
    p.t_dvs = p.add(ar, 4 * n * NP);
    p.t_dmix = p.add(ar, 4 * n * CN);
    p.t_ddir0 = p.add(ar, 4 * n * CN);
    p.t_ddir1 = p.add(ar, 4 * n * CN);
    p.t_dz = p.add(ar, 4 * n * H);
    p.t_dh0 = p.add(ar, 4 * n * H);
    p.t_dh1 = p.add(ar, 4 * n * H);
    return p;
}

static EqArgs eq_args(ModelImpl &m, MessagePlan &p, const Records &r, int b) {
    const rune_model_config &c = m.cfg;
    const BlockBuffers &bb = p.blocks[b];
    EqArgs a{};
    a.r = r;
    a.H = c.hidden_dim;
    a.D = c.message_dim;
    a.G = c.message_groups;
    a.C = c.equivariant_channels;
    a.lq = c.equivariant_l_max;
    a.nq = a.lq * (a.lq + 2);
    a.NG = a.G + 2 * a.lq * a.C;
    a.NP = 2 * a.D + a.H;
    a.kb = c.message_basis_size;
    a.na = m.desc.na;
    a.nlm = m.desc.nlm;
    a.S = eq_slots(a.C);
    {
        const int gw = a.H / a.G, cpl = a.H / 32;
        const bool pow2 = (gw & (gw - 1)) == 0;
        const int lpg = cpl > 0 ? gw / cpl : 0;
        const bool chunked = a.H % 32 == 0 && (cpl == 4 || cpl == 8 || cpl == 16) &&
                             gw % cpl == 0 && lpg >= 1 && (lpg & (lpg - 1)) == 0 &&
                             (2 * a.D + a.H) % 4 == 0 && a.NP % 4 == 0;
        a.gmode = chunked ? 3 : (pow2 && gw <= kWave) ? 0 : (gw % kWave == 0 ? 1 : 2);
    }
    a.eps = float(c.norm_eps);
    a.cutoff = float(c.message_cutoff);
    a.fc = p.at(p.i_fc);
    a.tfc = p.at(p.i_tfc);
    a.harm = p.at(p.i_harm);
    a.rb = p.at(p.i_rb);
    a.ldrb = p.ldrb;
    a.node = p.at(bb.vs);
    a.dir_in = p.at(bb.dir_in);
    a.dir_out = p.at(bb.dir_out);
    a.mixw = m.msg[b].mix;
    a.mixst = p.at(bb.mixstate);
    a.act = c.activation;
    a.pair = reinterpret_cast<const int32_t *>(p.at(p.i_pair));
    a.pair_proj = m.msg[b].pair_proj;
    a.wpc = m.msg[b].probe_c;
    a.wpn = m.msg[b].probe_n;
    a.wrb = m.msg[b].edge_rbT;
    a.ue = p.at(bb.ue);
    a.ldd = p.ld_edge;
    a.eh = p.at(bb.eh);
    a.ag = p.at(bb.gv);
    a.msg = p.at(bb.msg);
    a.rm = p.at(bb.rm);
    a.uin = p.at(bb.uin);
    a.duin = p.at(p.t_duin);
    a.dmsg = p.at(p.t_dmsg);
    a.dht = p.at(p.t_dvsum);
    a.dgg = p.at(p.t_dgv);
    a.dv = reinterpret_cast<float4 *>(p.at(p.i_dv));
    a.dfc = p.at(p.i_dfc);
    a.dy = p.at(p.i_dharm);
    a.dy_old = a.dy;
    a.dnode = p.at(p.t_dvs);
    a.dmix = p.at(p.t_dmix);
    a.due = p.at(p.t_due);
    a.qbuf = p.at(bb.q);
    a.dqbuf = p.at(p.t_dq);
    return a;
}

// The record-only forward work of the EQ blocks: edge features and
// harmonics, the cutoff of every transposed record, and the clearing of the
// dE/dfc accumulators and the zero row (no node state read).  dE/dY needs no
// clearing: the first reverse block writes every row.
void equivariant_record_forward(ModelImpl &m, MessagePlan &p, const Records &r,
                                const int32_t *types, hipStream_t s) {
    const rune_model_config &c = m.cfg;
    const int lq = c.equivariant_l_max, nq = lq * (lq + 2);
    const int64_t E = p.E;
    {
        Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
        edge_prep(m, p, r, types, s, p.at(p.i_harm), m.harm_scale, lq, nq);
    }
    Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
    hipLaunchKernelGGL(k_gather_f, dim3(ceil_div(std::max<int64_t>(E, 128), 256)), dim3(256), 0,
                       s, E, r.tidx, p.at(p.i_fc), p.at(p.i_tfc), p.at(p.i_dfc), p.at(p.i_zero),
                       128);
    RUNE_HIP_CHECK(hipGetLastError());
}

float *equivariant_forward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                           const int32_t *types, const float *moments, float *h, hipStream_t s,
                           bool keep) {
    (void)lp;
    (void)keep;
    const rune_model_config &c = m.cfg;
    const int N = p.N, H = c.hidden_dim, D = c.message_dim, act = c.activation;
    const int lq = c.equivariant_l_max, C = c.equivariant_channels, nq = lq * (lq + 2);
    const int64_t E = p.E;
    const int atom_grid = ceil_div(N, kWaves), mix_grid = std::max(1, std::min(ceil_div(N, 4), 4096));
    if (!p.records_ready) equivariant_record_forward(m, p, r, types, s);
    {
        const int wrow = (std::max(m.desc.na * m.desc.nlm, C * nq) + 3) & ~3;
        const size_t lds = sizeof(float) * (size_t(lq) * C * m.desc.na + 4 * size_t(wrow));
        hipLaunchKernelGGL(k_eq_encode, dim3(mix_grid), dim3(256), lds, s, N, moments, m.desc.na,
                           m.desc.nlm, m.enc_w, m.harm_scale, lq, C, nq, wrow,
                           p.at(p.blocks[0].dir_in));
    }
    RUNE_HIP_CHECK(hipGetLastError());
    const float *cur = h;
    for (int b = 0; b < c.message_layers; ++b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        EqArgs a = eq_args(m, p, r, b);
        Epilogue e0;
        e0.rms_out = p.at(bb.rin);   // input RMSNorm, formed by the GEMM
        e0.rms_eps = float(c.norm_eps);
        gemm(N, w.NP, H, cur, H, w.node_f, H, p.at(bb.vs), w.NP, e0, s);
        launch_mix(lq, C, N, w.mix, p.at(bb.dir_in), 0, nullptr, nullptr, p.at(bb.mixstate), s);
        if (E > 0) {
            const int dmc = edge_dmc(lq, D), cn4 = (C * nq + 3) & ~3;
            const int ly = nq + (nq % 4 == 0 ? 4 : 1);
            const dim3 egrid(atom_grid, ceil_div(D, kWave * dmc));
            {
                Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
                // per-wave record rows, or (prologue) the state rows plus one
                // order's weight chunk
                const int pro = ceil_div(kWaves * cn4 + C * kWave * dmc, kWaves);
                // a multiple of 4 floats: the record rows are read as 16-byte vectors
                a.wlds = (std::max({cn4, kWave * (ly + std::max(p.ldrb, kRcStride)), pro}) + 3) & ~3;
                const size_t lds_n = sizeof(float) * kWaves * a.wlds;
                EQ_LAUNCH_D(k_eq_edge_nbr, lq, dmc, egrid, dim3(kBlock), lds_n, s, a);
            }
            {
                Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
                const int pro = ceil_div(kWaves * cn4 + C * kWave * dmc, kWaves);
                a.wlds = (std::max({cn4, kWave * ly, pro}) + 3) & ~3;
                const size_t lds_c = sizeof(float) * kWaves * a.wlds;
                EQ_LAUNCH_D(k_eq_edge_centre, lq, dmc, egrid, dim3(kBlock), lds_c, s, a);
            }
            Epilogue e2;
            e2.bias = w.gate_b;
            e2.act = kActSigmoid;
            e2.act_split = c.message_groups;
            e2.act2 = RUNE_ACT_TANH;
            {
                Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                gemm(int(E), w.NG, D, p.at(bb.eh), p.ld_edge, w.gate, D, p.at(bb.gv), w.NG, e2,
                     s);
            }
        }
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            EQ_LAUNCH_S(k_eq_aggregate, lq, a.S, dim3(atom_grid), dim3(kBlock),
                        sizeof(float) * kBlock * (nq + (nq % 4 == 0 ? 4 : 1)), s, a);
        }
        const int NU = H + lq * C;
        Epilogue e3;
        e3.bias = w.up1_b;
        e3.pre = p.at(bb.u1);
        e3.ldp = D;
        e3.act = act;
        gemm(N, D, NU, p.at(bb.uin), NU, w.up1_f, NU, p.at(bb.z1), D, e3, s);
        Epilogue e4;
        e4.bias = w.up2_b;
        e4.residual = cur;
        e4.ldr = H;
        gemm(N, H, D, p.at(bb.z1), D, w.up2, D, p.at(bb.h_out), H, e4, s);
        p.block_input.push_back(cur);
        cur = p.at(bb.h_out);
    }
    return const_cast<float *>(cur);
}

float *equivariant_backward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                            const int32_t *types, const float *moments, float *dh,
                            hipStream_t s) {
    (void)lp;
    (void)types;
    (void)moments;
    const rune_model_config &c = m.cfg;
    const int N = p.N, H = c.hidden_dim, D = c.message_dim, act = c.activation;
    const int lq = c.equivariant_l_max, C = c.equivariant_channels, nq = lq * (lq + 2);
    const int NU = H + lq * C, kb = c.message_basis_size, ldd = p.ld_edge;
    const int64_t E = p.E;
    const int atom_grid = ceil_div(N, kWaves), mix_grid = std::max(1, std::min(ceil_div(N, 4), 4096));
    const int ly = nq + (nq % 4 == 0 ? 4 : 1);
    const int ntc = adj_ntc(lq, ldd), mt = (nq + 16) / 16;
    // per-wave LDS of the reverse edge-MLP kernels: due, harmonic and old dE/dY
    // rows of one batch, and its record ids
    const int adj_wlds = kAdjBatch * ((16 * ntc + 4) + (16 * mt + 4) + (nq + 1) + 1);
    float *cur = dh;
    const float *ddir_out = nullptr;   // the last block's states feed only its invariants
    float *ddir_in = p.at(p.t_ddir0);
    for (int b = c.message_layers - 1; b >= 0; --b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        EqArgs a = eq_args(m, p, r, b);
        if (b == c.message_layers - 1) a.dy_old = p.at(p.i_zero);
        a.ddir_out = ddir_out;
        a.ddir_in = ddir_in;
        Epilogue e0;
        e0.dact_from = p.at(bb.u1);
        e0.ldu = D;
        e0.dact = act;
        gemm(N, D, H, cur, H, w.up2_T, H, p.at(p.t_dz1), D, e0, s);
        Epilogue e1;
        gemm(N, NU, D, p.at(p.t_dz1), D, w.up1_fT, D, p.at(p.t_duin), NU, e1, s);
        hipLaunchKernelGGL(k_eq_node_backward, dim3(N), dim3(kWave), 0, s, a);
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            const size_t lds_pd = sizeof(float) * kWaves *
                                  (pair_dir_chunk(nq) * ly + a.S * nq * (kWave / a.S + 4));
            EQ_LAUNCH_S(k_eq_pair_dir, lq, a.S, dim3(atom_grid), dim3(kBlock), lds_pd, s, a);
        }
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            if (a.gmode == 3) {
                if (H == 128)
                    hipLaunchKernelGGL(k_eq_pair_grp_c<4>, dim3(atom_grid), dim3(kBlock), 0, s, a);
                else if (H == 256)
                    hipLaunchKernelGGL(k_eq_pair_grp_c<8>, dim3(atom_grid), dim3(kBlock), 0, s, a);
                else
                    hipLaunchKernelGGL(k_eq_pair_grp_c<16>, dim3(atom_grid), dim3(kBlock), 0, s, a);
            } else {
                hipLaunchKernelGGL(k_eq_pair_grp, dim3(atom_grid), dim3(kBlock),
                                   a.gmode == 2 ? sizeof(float) * kWaves * H : 0, s, a);
            }
        }
        RUNE_HIP_CHECK(hipGetLastError());
        if (E > 0) {
            // due = (dE/dgates) gate^T * act'(u), zero in the padding columns
            Epilogue e2;
            e2.dact_from = p.at(bb.ue);
            e2.ldu = ldd;
            e2.dact = act;
            {
                Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                gemm(int(E), ldd, w.NG, p.at(p.t_dgv), w.NG, w.gate_Tp, w.NG, p.at(p.t_due), ldd,
                     e2, s);
            }
            // dE/drb = due W_rb^T, summed over the blocks
            Epilogue e3;
            if (b != c.message_layers - 1) {
                e3.residual = p.at(p.i_drb);
                e3.ldr = p.ldrb;
            }
            {
                Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                gemm(int(E), kb, D, p.at(p.t_due), ldd, w.edge_rbT, D, p.at(p.i_drb), p.ldrb, e3,
                     s);
            }
        }
        a.wlds = adj_wlds;
        for (int side = 0; side < 2; ++side) {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            const size_t lds = sizeof(float) * kWaves * adj_wlds;
            if (side == 0)
                EQ_LAUNCH_A(k_eq_edge_adj, lq, ntc, 0, dim3(atom_grid), dim3(kBlock), lds, s, a);
            else
                EQ_LAUNCH_A(k_eq_edge_adj, lq, ntc, 1, dim3(atom_grid), dim3(kBlock), lds, s, a);
        }
        // channel projection of the factor adjoints: dHk[n, k, :] = dQ[n, k, :] [Wc | Wn]_L(k)^T
        {
            GemmBatch bt;
            bt.count = nq;
            bt.sa = 2 * int64_t(ldd);
            bt.sb = int64_t(C) * 2 * ldd;
            bt.sc = C;
            bt.b_by_order = 1;
            gemm_batched(bt, N, C, 2 * ldd, p.at(p.t_dq), nq * 2 * ldd, w.probe_cat, 2 * ldd,
                         p.at(p.t_dhk), nq * C, s);
        }
        // dE/d(dir_in) = M^T dmix + dE/d(dir_out) + the factor adjoints
        launch_mix(lq, C, N, w.mix, a.dmix, 1, p.at(p.t_dvsum), p.at(p.t_dhk), a.ddir_in, s);
        Epilogue e4;
        gemm(N, H, w.NP, p.at(p.t_dvs), w.NP, w.node_fT, w.NP, p.at(p.t_dz), H, e4, s);
        float *next = (cur == p.at(p.t_dh0)) ? p.at(p.t_dh1) : p.at(p.t_dh0);
        rms_backward(N, H, p.block_input[b], H, p.at(bb.rin), p.at(p.t_dz), H, cur, H, next, H, s);
        cur = next;
        ddir_out = ddir_in;
        ddir_in = (ddir_in == p.at(p.t_ddir0)) ? p.at(p.t_ddir1) : p.at(p.t_ddir0);
    }
    // ddir_out now holds dE/d(encoder output)
    {
        const int wrow = (std::max(m.desc.na * m.desc.nlm, C * nq) + 3) & ~3;
        const size_t lds = sizeof(float) * (size_t(lq) * C * m.desc.na + 4 * size_t(wrow));
        hipLaunchKernelGGL(k_eq_encoder_backward, dim3(mix_grid), dim3(256), lds, s, N, ddir_out,
                           m.enc_w, m.harm_scale, lq, C, nq, m.desc.na, m.desc.nlm, wrow, p.dmom);
    }
    if (E > 0) {
        EdgeZ zo;
        for (int k = 0; k < kMaxL + 2; ++k) zo.off[k] = m.desc.z_off[k];
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            EQ_LAUNCH(k_eq_harmonic_backward, lq, dim3(ceil_div(E, 256)), dim3(256), 0, s, E, r,
                      p.at(p.i_fc), p.at(p.i_dharm), p.at(p.i_dfc),
                      p.at(p.i_drb), p.at(p.i_rbd), p.ldrb, kb, float(c.message_cutoff),
                      m.desc.z, zo, m.harm_scale, reinterpret_cast<float4 *>(p.at(p.i_dv)));
        }
    }
    RUNE_HIP_CHECK(hipGetLastError());
    {
        Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
        edge_direct(p, r, s);
    }
    p.g_direct_used = E > 0;
    p.dmom_used = true;
    return cur;
}

}  // namespace rune
