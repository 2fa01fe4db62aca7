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
#include <cmath>

#include "message.hpp"

namespace rune {
namespace {

constexpr int kWave = 64;
constexpr float kPi = 3.14159265358979323846f;
constexpr int kMaxOut = 12;   // C * nq <= 768 outputs per atom, 12 per lane

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ inline int order_of(int k) {
    int L = 1;
    while ((L + 1) * (L + 1) - 1 <= k) ++L;
    return L;
}

struct EqArgs {
    Records r;
    int H, D, G, C, lq, nq, NG, NP, KX, kb, ldx, na, nlm;
    float eps, cutoff;
    const float *fc;          // [E]
    const float *harm;        // [E, nq]
    const float *rb;          // [E, ldrb]
    int ldrb;
    const float *node;        // [N, NP] = A | B | V
    const float *dir_in;      // [N, C*nq]
    float *dir_out;           // [N, C*nq]
    const float *mixw;        // [lq, C, C]
    float *mixst;             // [N, C*nq] channel-mixed dir_in
    float *x;                 // [E, ldx] edge features
    const float *ag;          // [E, NG] activated gates (sigmoid | tanh)
    float *msg, *rm, *uin;    // [N, H], [N], [N, H + lq*C]
    // reverse
    const float *duin;        // [N, H + lq*C]
    float *dmsg;              // [N, H]
    float *dht;               // [N, C*nq] dE/d(dir_out), total
    const float *ddir_out;    // [N, C*nq] from later blocks, or null
    float *dgg;               // [E, NG]
    float4 *dv;               // [E]
    float *dy;                // [E, nq]
    float *dnode;             // [N, NP]
    float *dmix;              // [N, C*nq]
    const float *due;         // [E, D]
    const float *dx;          // [E, ldx]
    float *ddir_in;           // [N, C*nq]
};

__global__ void __launch_bounds__(kWave) k_eq_encode(int N, const float *s, int na, int nlm,
                                                     const float *enc, const float *scale,
                                                     int C, int nq, float *out) {
    const int i = blockIdx.x, lane = threadIdx.x;
    for (int o = lane; o < C * nq; o += kWave) {
        int c = o / nq, k = o - c * nq, L = order_of(k);
        const float *w = enc + size_t((L - 1) * C + c) * na;
        float acc = 0.0f;
        for (int n = 0; n < na; ++n) acc += w[n] * (s[size_t(i) * na * nlm + n * nlm + k] * scale[k]);
        out[size_t(i) * C * nq + o] = acc;
    }
}

__global__ void __launch_bounds__(kWave) k_eq_mix(const float *mixw, const float *in, int C,
                                                  int nq, float *out) {
    const int i = blockIdx.x, lane = threadIdx.x;
    const float *h = in + size_t(i) * C * nq;
    for (int o = lane; o < C * nq; o += kWave) {
        int c = o / nq, k = o - c * nq, L = order_of(k);
        const float *M = mixw + size_t((L - 1) * C + c) * C;
        float acc = 0.0f;
        for (int cc = 0; cc < C; ++cc) acc += M[cc] * h[cc * nq + k];
        out[size_t(i) * C * nq + o] = acc;
    }
}

// Per-edge loops.  Each kernel walks the records of one atom in chunks of 64:
// the chunk's record metadata (neighbour / centre index, cutoff value) is read
// lane-parallel once and broadcast per record with readlane, and the rows of
// the next record are fetched into registers while the current one is
// processed, so no record waits on a chain of dependent loads.
__device__ inline int lane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ inline float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

constexpr int kMaxG = 9;     // NG <= 64 + 2 * 256 gate columns, 9 per lane
constexpr int kMaxY = 1;     // nq <= 64 harmonic components, 1 per lane

// Edge features [rb | probes_c | probes_n] of the radial records of centre i.
__global__ void __launch_bounds__(kWave) k_eq_features(EqArgs a) {
    extern __shared__ float lds[];
    const int C = a.C, nq = a.nq, lq = a.lq, LC = lq * C, CN = C * nq;
    const int ldc = nq | 1;   // odd LDS row stride: channel-strided reads hit distinct banks
    float *Hi = lds;          // [C][ldc] centre state
    float *Hj = Hi + C * ldc; // [C][ldc] neighbour state of the current record
    float *Yl = Hj + C * ldc; // [nq]
    const int i = blockIdx.x, lane = threadIdx.x;
    int so[kMaxOut];
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        int o = lane + kWave * t;
        so[t] = o < CN ? (o / nq) * ldc + o % nq : -1;
        if (so[t] >= 0) Hi[so[t]] = a.dir_in[size_t(i) * CN + o];
    }
    float hn[kMaxOut], yn = 0.0f, rn = 0.0f;
    auto fetch = [&](int e, int j) {
#pragma unroll
        for (int t = 0; t < kMaxOut; ++t)
            hn[t] = so[t] >= 0 ? a.dir_in[size_t(j) * CN + lane + kWave * t] : 0.0f;
        yn = lane < nq ? a.harm[size_t(e) * nq + lane] : 0.0f;
        rn = lane < a.kb ? a.rb[size_t(e) * a.ldrb + lane] : 0.0f;
    };
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int c0 = rb; c0 < re; c0 += kWave) {
        const int cnt = min(kWave, re - c0);
        int mj = 0;
        float mf = 0.0f;
        if (lane < cnt) {
            mj = a.r.nbr[c0 + lane];
            mf = a.fc[c0 + lane];
        }
        fetch(c0, lane_i(mj, 0));
        for (int u = 0; u < cnt; ++u) {
            const int e = c0 + u;
            const float fc = lane_f(mf, u);
            __syncthreads();
#pragma unroll
            for (int t = 0; t < kMaxOut; ++t)
                if (so[t] >= 0) Hj[so[t]] = hn[t];
            if (lane < nq) Yl[lane] = yn;
            const float rcur = rn;
            __syncthreads();
            if (u + 1 < cnt) fetch(e + 1, lane_i(mj, u + 1));
            float *x = a.x + size_t(e) * a.ldx;
            if (fc == 0.0f) {
                for (int k = lane; k < a.KX; k += kWave) x[k] = 0.0f;
                continue;
            }
            if (lane < a.kb) x[lane] = rcur;
            for (int p = lane; p < LC; p += kWave) {
                int L = p / C + 1, c = p - (L - 1) * C, st = L * L - 1;
                float pc = 0.0f, pn = 0.0f;
                for (int m = 0; m < 2 * L + 1; ++m) {
                    pc += Hi[c * ldc + st + m] * Yl[st + m];
                    pn += Hj[c * ldc + st + m] * Yl[st + m];
                }
                x[a.kb + p] = pc;
                x[a.kb + LC + p] = (L & 1) ? -pn : pn;
            }
        }
    }
}

// Messages and transported / injected direction states of centre i, then the
// update input [RMSNorm(msg) | per-(L, c) squared norms of dir_out].
__global__ void __launch_bounds__(kWave) k_eq_aggregate(EqArgs a) {
    extern __shared__ float lds[];
    const int H = a.H, G = a.G, C = a.C, nq = a.nq, lq = a.lq, gw = H / G, LC = lq * C;
    const int CN = C * nq, NG = a.NG;
    float *Ho = lds;          // [CN]
    float *gL = Ho + CN;      // [NG] gates of the current record
    float *Yl = gL + NG;      // [nq]
    const int i = blockIdx.x, lane = threadIdx.x;
    float macc[4] = {0, 0, 0, 0};
    float dacc[kMaxOut];
    int gT[kMaxOut], kk[kMaxOut];
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        dacc[t] = 0.0f;
        int o = lane + kWave * t;
        int c = o / nq, k = o - c * nq;
        kk[t] = k;
        gT[t] = o < CN ? G + (order_of(k) - 1) * C + c : 0;
    }
    float gn[kMaxG], vn[4], mxn[kMaxOut], yn = 0.0f;
    auto fetch = [&](int e, int j) {
#pragma unroll
        for (int q = 0; q < kMaxG; ++q) {
            int k = lane + kWave * q;
            gn[q] = k < NG ? a.ag[size_t(e) * NG + k] : 0.0f;
        }
        yn = lane < nq ? a.harm[size_t(e) * nq + lane] : 0.0f;
        const float *V = a.node + size_t(j) * a.NP + 2 * a.D;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int c = lane + kWave * t;
            vn[t] = c < H ? V[c] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < kMaxOut; ++t) {
            int o = lane + kWave * t;
            mxn[t] = o < CN ? a.mixst[size_t(j) * CN + o] : 0.0f;
        }
    };
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int c0 = rb; c0 < re; c0 += kWave) {
        const int cnt = min(kWave, re - c0);
        int mj = 0;
        float mf = 0.0f;
        if (lane < cnt) {
            mj = a.r.nbr[c0 + lane];
            mf = a.fc[c0 + lane];
        }
        fetch(c0, lane_i(mj, 0));
        for (int u = 0; u < cnt; ++u) {
            const float fc = lane_f(mf, u);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kMaxG; ++q)
                if (lane + kWave * q < NG) gL[lane + kWave * q] = gn[q];
            if (lane < nq) Yl[lane] = yn;
            float vc[4], mx[kMaxOut];
#pragma unroll
            for (int t = 0; t < 4; ++t) vc[t] = vn[t];
#pragma unroll
            for (int t = 0; t < kMaxOut; ++t) mx[t] = mxn[t];
            __syncthreads();
            if (u + 1 < cnt) fetch(c0 + u + 1, lane_i(mj, u + 1));
            if (fc == 0.0f) continue;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int c = lane + kWave * t;
                if (c < H) macc[t] += gL[c / gw] * fc * vc[t];
            }
#pragma unroll
            for (int t = 0; t < kMaxOut; ++t) {
                int o = lane + kWave * t;
                if (o < CN) dacc[t] += fc * (gL[gT[t]] * mx[t] + gL[gT[t] + LC] * Yl[kk[t]]);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        int o = lane + kWave * t;
        if (o < CN) {
            float v = a.dir_in[size_t(i) * CN + o] + dacc[t];
            a.dir_out[size_t(i) * CN + o] = v;
            Ho[o] = v;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        int c = lane + kWave * t;
        if (c < H) {
            a.msg[size_t(i) * H + c] = macc[t];
            ss += macc[t] * macc[t];
        }
    }
    ss = wave_sum(ss);
    float r = 1.0f / sqrtf(ss / float(H) + a.eps);
    if (lane == 0) a.rm[i] = r;
    const int ldu = H + LC;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        int c = lane + kWave * t;
        if (c < H) a.uin[size_t(i) * ldu + c] = macc[t] * r;
    }
    __syncthreads();
    for (int p = lane; p < LC; p += kWave) {
        int L = p / C + 1, c = p - (L - 1) * C, st = L * L - 1;
        float s = 0.0f;
        for (int m = 0; m < 2 * L + 1; ++m) s += Ho[c * nq + st + m] * Ho[c * nq + st + m];
        a.uin[size_t(i) * ldu + H + p] = s;
    }
}

__global__ void __launch_bounds__(kWave) k_eq_node_backward(EqArgs a) {
    const int i = blockIdx.x, lane = threadIdx.x;
    const int H = a.H, C = a.C, nq = a.nq, LC = a.lq * C, ldu = H + LC, CN = C * nq;
    const float *d = a.duin + size_t(i) * ldu;
    const float *m = a.msg + size_t(i) * H;
    float dot = 0.0f;
    for (int c = lane; c < H; c += kWave) dot += d[c] * m[c];
    dot = wave_sum(dot);
    float r = a.rm[i];
    float coef = r * r * r * dot / float(H);
    for (int c = lane; c < H; c += kWave) a.dmsg[size_t(i) * H + c] = r * d[c] - coef * m[c];
    for (int o = lane; o < CN; o += kWave) {
        int c = o / nq, k = o - c * nq, L = order_of(k);
        float g = a.ddir_out ? a.ddir_out[size_t(i) * CN + o] : 0.0f;
        g += 2.0f * a.dir_out[size_t(i) * CN + o] * d[H + (L - 1) * C + c];
        a.dht[size_t(i) * CN + o] = g;
    }
}

// Gate adjoints and dE/dfc for the records of centre i.
__global__ void __launch_bounds__(kWave) k_eq_edge_backward(EqArgs a) {
    extern __shared__ float lds[];
    const int H = a.H, G = a.G, C = a.C, nq = a.nq, lq = a.lq, gw = H / G, LC = lq * C;
    const int CN = C * nq, NG = a.NG, ldc = nq | 1;
    float *DH = lds;             // [C][ldc] dE/d(dir_out) of centre i
    float *MX = DH + C * ldc;    // [C][ldc] mixed state of the current neighbour
    float *pL = MX + C * ldc;    // [H] dmsg_i * V_j
    float *gL = pL + H;          // [NG]
    float *YL = gL + NG;         // [nq]
    const int i = blockIdx.x, lane = threadIdx.x;
    int so[kMaxOut];
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        int o = lane + kWave * t;
        so[t] = o < CN ? (o / nq) * ldc + o % nq : -1;
        if (so[t] >= 0) DH[so[t]] = a.dht[size_t(i) * CN + o];
    }
    float dm[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        int c = lane + kWave * t;
        dm[t] = c < H ? a.dmsg[size_t(i) * H + c] : 0.0f;
    }
    float gn[kMaxG], vn[4], mxn[kMaxOut], yn = 0.0f;
    auto fetch = [&](int e, int j) {
#pragma unroll
        for (int q = 0; q < kMaxG; ++q) {
            int k = lane + kWave * q;
            gn[q] = k < NG ? a.ag[size_t(e) * NG + k] : 0.0f;
        }
        yn = lane < nq ? a.harm[size_t(e) * nq + lane] : 0.0f;
        const float *V = a.node + size_t(j) * a.NP + 2 * a.D;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int c = lane + kWave * t;
            vn[t] = c < H ? V[c] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < kMaxOut; ++t)
            mxn[t] = so[t] >= 0 ? a.mixst[size_t(j) * CN + lane + kWave * t] : 0.0f;
    };
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int c0 = rb; c0 < re; c0 += kWave) {
        const int cnt = min(kWave, re - c0);
        int mj = 0;
        float mf = 0.0f;
        if (lane < cnt) {
            mj = a.r.nbr[c0 + lane];
            mf = a.fc[c0 + lane];
        }
        fetch(c0, lane_i(mj, 0));
        for (int u = 0; u < cnt; ++u) {
            const int e = c0 + u;
            const float fc = lane_f(mf, u);
            float *dg = a.dgg + size_t(e) * NG;
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kMaxG; ++q)
                if (lane + kWave * q < NG) gL[lane + kWave * q] = gn[q];
            if (lane < nq) YL[lane] = yn;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int c = lane + kWave * t;
                if (c < H) pL[c] = dm[t] * vn[t];
            }
#pragma unroll
            for (int t = 0; t < kMaxOut; ++t)
                if (so[t] >= 0) MX[so[t]] = mxn[t];
            __syncthreads();
            if (u + 1 < cnt) fetch(e + 1, lane_i(mj, u + 1));
            if (fc == 0.0f) {
                for (int k = lane; k < NG; k += kWave) dg[k] = 0.0f;
                continue;
            }
            float dfc = 0.0f;
            for (int p = lane; p < LC; p += kWave) {
                int L = p / C + 1, c = p - (L - 1) * C, st = L * L - 1;
                float sT = 0.0f, sI = 0.0f;
                for (int m = 0; m < 2 * L + 1; ++m) {
                    float d = DH[c * ldc + st + m];
                    sT += d * MX[c * ldc + st + m];
                    sI += d * YL[st + m];
                }
                float tT = gL[G + p], tI = gL[G + LC + p];
                dg[G + p] = (1.0f - tT * tT) * fc * sT;
                dg[G + LC + p] = (1.0f - tI * tI) * fc * sI;
                dfc += tT * sT + tI * sI;
            }
            if (lane < G) {
                float P = 0.0f;
                for (int c = lane * gw; c < (lane + 1) * gw; ++c) P += pL[c];
                float s = gL[lane];
                dg[lane] = P * fc * s * (1.0f - s);
                dfc += P * s;
            }
            dfc = wave_sum(dfc);
            if (lane == 0) {
                float d = a.r.vec[e].w;
                float fcp = -0.5f * kPi / a.cutoff * sinf(kPi * d / a.cutoff);
                a.dv[e].w += dfc * fcp;
            }
        }
    }
}

// Adjoints landing on neighbour j: mixed states and gathered values.
__global__ void __launch_bounds__(kWave) k_eq_neighbor_backward(EqArgs a) {
    extern __shared__ float gL[];   // [NG] gates of the current record
    const int j = blockIdx.x, lane = threadIdx.x;
    const int H = a.H, G = a.G, C = a.C, nq = a.nq, gw = H / G, CN = C * nq, NG = a.NG;
    float macc[kMaxOut];
    int gT[kMaxOut];
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        macc[t] = 0.0f;
        int o = lane + kWave * t;
        int c = o / nq, k = o - c * nq;
        gT[t] = o < CN ? G + (order_of(k) - 1) * C + c : 0;
    }
    float vacc[4] = {0, 0, 0, 0};
    float gn[kMaxG], dhn[kMaxOut], dmn[4];
    auto fetch = [&](int e, int i) {
#pragma unroll
        for (int q = 0; q < kMaxG; ++q) {
            int k = lane + kWave * q;
            gn[q] = k < NG ? a.ag[size_t(e) * NG + k] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < kMaxOut; ++t) {
            int o = lane + kWave * t;
            dhn[t] = o < CN ? a.dht[size_t(i) * CN + o] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int c = lane + kWave * t;
            dmn[t] = c < H ? a.dmsg[size_t(i) * H + c] : 0.0f;
        }
    };
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    for (int c0 = tb; c0 < te; c0 += kWave) {
        const int cnt = min(kWave, te - c0);
        int me = 0, mi = 0;
        float mf = 0.0f;
        if (lane < cnt) {
            me = a.r.tidx[c0 + lane];
            mi = a.r.ctr[me];
            mf = a.fc[me];
        }
        fetch(lane_i(me, 0), lane_i(mi, 0));
        for (int u = 0; u < cnt; ++u) {
            const float fc = lane_f(mf, u);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kMaxG; ++q)
                if (lane + kWave * q < NG) gL[lane + kWave * q] = gn[q];
            float dh[kMaxOut], dmc[4];
#pragma unroll
            for (int t = 0; t < kMaxOut; ++t) dh[t] = dhn[t];
#pragma unroll
            for (int t = 0; t < 4; ++t) dmc[t] = dmn[t];
            __syncthreads();
            if (u + 1 < cnt) fetch(lane_i(me, u + 1), lane_i(mi, u + 1));
            if (fc == 0.0f) continue;
#pragma unroll
            for (int q = 0; q < kMaxOut; ++q) {
                int o = lane + kWave * q;
                if (o < CN) macc[q] += fc * gL[gT[q]] * dh[q];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int c = lane + kWave * q;
                if (c < H) vacc[q] += gL[c / gw] * fc * dmc[q];
            }
        }
    }
#pragma unroll
    for (int q = 0; q < kMaxOut; ++q) {
        int o = lane + kWave * q;
        if (o < CN) a.dmix[size_t(j) * CN + o] = macc[q];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        int c = lane + kWave * q;
        if (c < H) a.dnode[size_t(j) * a.NP + 2 * a.D + c] = vacc[q];
    }
}

// Per-atom adjoints: context projections A (own records) and B (as neighbour),
// and dE/d(dir_in) = identity + probes + channel mix.
__global__ void __launch_bounds__(kWave) k_eq_atom_backward(EqArgs a) {
    extern __shared__ float lds[];
    const int C = a.C, nq = a.nq, lq = a.lq, LC = lq * C, CN = C * nq, D = a.D;
    float *dxL = lds;          // [LC] probe adjoints of the current record
    float *Yl = dxL + LC;      // [nq]
    float *dmixL = Yl + nq;    // [CN]
    const int n = blockIdx.x, lane = threadIdx.x;
    float sa[4] = {0, 0, 0, 0}, sb[4] = {0, 0, 0, 0};
    float g[kMaxOut];
    int col[kMaxOut], kk[kMaxOut], LL[kMaxOut];
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        int o = lane + kWave * t;
        int c = o / nq, k = o - c * nq, L = o < CN ? order_of(k) : 1;
        kk[t] = k;
        LL[t] = L;
        col[t] = (L - 1) * C + c;
        g[t] = o < CN ? a.dht[size_t(n) * CN + o] : 0.0f;
    }
    float dun[4], dxn[4], yn = 0.0f;
    auto fetch = [&](int e, int off) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int c = lane + kWave * q;
            dun[q] = c < D ? a.due[size_t(e) * D + c] : 0.0f;
            dxn[q] = c < LC ? a.dx[size_t(e) * a.ldx + a.kb + off + c] : 0.0f;
        }
        yn = lane < nq ? a.harm[size_t(e) * nq + lane] : 0.0f;
    };
    // own records: dA, probes_c adjoint (sign +1); records as neighbour: dB,
    // probes_n adjoint (sign (-1)^L)
    for (int side = 0; side < 2; ++side) {
        const int b0 = side ? a.r.tptr[n] : a.r.view[4 * n];
        const int b1 = side ? a.r.tptr[n + 1] : a.r.view[4 * n + 1];
        for (int c0 = b0; c0 < b1; c0 += kWave) {
            const int cnt = min(kWave, b1 - c0);
            int me = 0;
            float mf = 0.0f;
            if (lane < cnt) {
                me = side ? a.r.tidx[c0 + lane] : c0 + lane;
                mf = a.fc[me];
            }
            fetch(lane_i(me, 0), side * LC);
            for (int u = 0; u < cnt; ++u) {
                const float fc = lane_f(mf, u);
                __syncthreads();
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (lane + kWave * q < LC) dxL[lane + kWave * q] = dxn[q];
                if (lane < nq) Yl[lane] = yn;
                float du[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) du[q] = dun[q];
                __syncthreads();
                if (u + 1 < cnt) fetch(lane_i(me, u + 1), side * LC);
                if (fc == 0.0f) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (side)
                        sb[q] += du[q];
                    else
                        sa[q] += du[q];
                }
#pragma unroll
                for (int t = 0; t < kMaxOut; ++t)
                    if (lane + kWave * t < CN) {
                        float v = dxL[col[t]] * Yl[kk[t]];
                        g[t] += (side && (LL[t] & 1)) ? -v : v;
                    }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        int c = lane + kWave * q;
        if (c < D) {
            a.dnode[size_t(n) * a.NP + c] = sa[q];
            a.dnode[size_t(n) * a.NP + D + c] = sb[q];
        }
    }
    // channel mix adjoint: dH[c][k] += sum_c' M_L[c'][c] dMIX[c'][k]
    __syncthreads();
    for (int o = lane; o < CN; o += kWave) dmixL[o] = a.dmix[size_t(n) * CN + o];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        int o = lane + kWave * t;
        if (o >= CN) continue;
        int c = col[t] - (LL[t] - 1) * C;
        const float *M = a.mixw + size_t(LL[t] - 1) * C * C + c;
        float s = 0.0f;
        for (int cc = 0; cc < C; ++cc) s += M[cc * C] * dmixL[cc * nq + kk[t]];
        a.ddir_in[size_t(n) * CN + o] = g[t] + s;
    }
}

// dE/dY of the records of centre i: the injected direction term
// fc tI[L,c] dHt_i[c][k] and the probes of the centre and neighbour states.
__global__ void __launch_bounds__(kWave) k_eq_probe_dy(EqArgs a) {
    extern __shared__ float lds[];
    const int C = a.C, nq = a.nq, LC = a.lq * C, CN = C * nq, G = a.G, NG = a.NG;
    const int ldc = nq | 1;
    float *Hi = lds;             // [C][ldc]
    float *DH = Hi + C * ldc;    // [C][ldc]
    float *Hj = DH + C * ldc;    // [C][ldc]
    float *cf = Hj + C * ldc;    // [3 LC] injection gates | centre / neighbour probe adjoints
    const int i = blockIdx.x, lane = threadIdx.x;
    int so[kMaxOut];
#pragma unroll
    for (int t = 0; t < kMaxOut; ++t) {
        int o = lane + kWave * t;
        so[t] = o < CN ? (o / nq) * ldc + o % nq : -1;
        if (so[t] >= 0) {
            Hi[so[t]] = a.dir_in[size_t(i) * CN + o];
            DH[so[t]] = a.dht[size_t(i) * CN + o];
        }
    }
    // contraction layout: component k = lane % nq, channels c = cg, cg + ncg, ...
    const int ncg = kWave / nq, k = lane % nq, cg = lane / nq, L = order_of(k);
    float hn[kMaxOut], cn[kMaxOut];
    auto fetch = [&](int e, int j) {
#pragma unroll
        for (int t = 0; t < kMaxOut; ++t)
            hn[t] = so[t] >= 0 ? a.dir_in[size_t(j) * CN + lane + kWave * t] : 0.0f;
#pragma unroll
        for (int t = 0; t < kMaxOut; ++t) {
            int q = lane + kWave * t;
            float v = 0.0f;
            if (q < LC)
                v = a.ag[size_t(e) * NG + G + LC + q];
            else if (q < 3 * LC)
                v = a.dx[size_t(e) * a.ldx + a.kb + q - LC];
            cn[t] = v;
        }
    };
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int c0 = rb; c0 < re; c0 += kWave) {
        const int cnt = min(kWave, re - c0);
        int mj = 0;
        float mf = 0.0f;
        if (lane < cnt) {
            mj = a.r.nbr[c0 + lane];
            mf = a.fc[c0 + lane];
        }
        fetch(c0, lane_i(mj, 0));
        for (int u = 0; u < cnt; ++u) {
            const int e = c0 + u;
            const float fc = lane_f(mf, u);
            __syncthreads();
#pragma unroll
            for (int t = 0; t < kMaxOut; ++t) {
                if (so[t] >= 0) Hj[so[t]] = hn[t];
                if (lane + kWave * t < 3 * LC) cf[lane + kWave * t] = cn[t];
            }
            __syncthreads();
            if (u + 1 < cnt) fetch(e + 1, lane_i(mj, u + 1));
            if (fc == 0.0f) continue;
            float y = 0.0f;
            if (cg < ncg) {
                const float *ti = cf + (L - 1) * C, *dc = ti + LC, *dn = ti + 2 * LC;
                float yi = 0.0f, yc = 0.0f, yn = 0.0f;
                for (int c = cg; c < C; c += ncg) {
                    yi += ti[c] * DH[c * ldc + k];
                    yc += dc[c] * Hi[c * ldc + k];
                    yn += dn[c] * Hj[c * ldc + k];
                }
                y = fc * yi + yc + ((L & 1) ? -yn : yn);
            }
            for (int s2 = 1; s2 < ncg; ++s2) {
                float v = __shfl(y, min(lane + s2 * nq, kWave - 1), kWave);
                if (cg == 0) y += v;
            }
            if (cg == 0) a.dy[size_t(e) * nq + k] += y;
        }
    }
}

__global__ void __launch_bounds__(kWave) k_eq_encoder_backward(const float *ddir0,
                                                               const float *enc,
                                                               const float *scale, int C,
                                                               int nq, int na, int nlm,
                                                               float *dmom) {
    const int i = blockIdx.x, lane = threadIdx.x;
    for (int o = lane; o < na * nlm; o += kWave) {
        int n = o / nlm, k = o - n * nlm;
        float g = 0.0f;
        if (k < nq) {
            int L = order_of(k);
            for (int c = 0; c < C; ++c)
                g += enc[size_t((L - 1) * C + c) * na + n] * ddir0[size_t(i) * C * nq + c * nq + k];
            g *= scale[k];
        }
        dmom[size_t(i) * na * nlm + o] = g;
    }
}

// dE/du of the harmonics: sum_k dY_k scale_k db_k/du, added to dv.xyz.
__global__ void k_eq_harmonic_backward(int64_t E, Records r, const float *fcv, const float *dy,
                                       const float *ztab, EdgeZ zoff, int lq, int nq,
                                       const float *scale, float4 *dv) {
    int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    int i = r.ctr[e];
    if (!(e >= r.view[4 * i] && e < r.view[4 * i + 1])) return;
    float4 v = r.vec[e];
    float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
    float x = v.x * inv, y = v.y * inv, z = v.z * inv;
    float zp[kMaxL + 1], wr[kMaxL + 1], wi[kMaxL + 1];
    zp[0] = 1.0f;
    wr[0] = 1.0f;
    wi[0] = 0.0f;
    for (int k = 1; k <= lq; ++k) {
        zp[k] = zp[k - 1] * z;
        wr[k] = wr[k - 1] * x - wi[k - 1] * y;
        wi[k] = wr[k - 1] * y + wi[k - 1] * x;
    }
    const float *g = dy + size_t(e) * nq;
    float dx = 0.0f, dyy = 0.0f, dz = 0.0f;
    int idx = 0;
    for (int L = 1; L <= lq; ++L) {
        for (int n1 = 0; n1 <= L; ++n1) {
            const float *Z = ztab + zoff.off[L] + n1 * (L + 1);
            float zf = 0.0f, zfp = 0.0f;
            for (int q = ((L + n1) & 1); q <= L - n1; q += 2) {
                zf += Z[q] * zp[q];
                if (q > 0) zfp += float(q) * Z[q] * zp[q - 1];
            }
            for (int part = 0; part < (n1 == 0 ? 1 : 2); ++part, ++idx) {
                float w = g[idx] * scale[idx];
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
    dv[e] = acc;
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static void expect(ModelImpl &m, const std::string &name, int64_t n) { m.expected[name] = n; }

void validate_equivariant(ModelImpl &m) {
    const rune_model_config &c = m.cfg;
    const int lq = c.equivariant_l_max, C = c.equivariant_channels;
    RUNE_REQUIRE(lq >= 1 && lq <= std::min(c.l_max, 7), RUNE_ERR_ARGUMENT,
                 "equivariant blocks support equivariant_l_max in 1..min(l_max, 7)");
    RUNE_REQUIRE(C >= 1 && C * lq * (lq + 2) <= kWave * kMaxOut, RUNE_ERR_ARGUMENT,
                 "equivariant_channels * l(l+2) must not exceed 768");
    RUNE_REQUIRE(c.message_groups <= kWave, RUNE_ERR_ARGUMENT, "message_groups must be <= 64");
    RUNE_REQUIRE(c.message_dim <= 4 * kWave, RUNE_ERR_ARGUMENT,
                 "equivariant blocks support message_dim <= 256");
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
    const int K = kb + P + 2 * D + 2 * W, NP = 2 * D + H, NG = G + 2 * W, KX = kb + 2 * W;
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
        std::vector<float> wx = columns(we, D, K, 0, kb);                    // [D, KX]
        std::vector<float> wp = columns(we, D, K, kb + P + 2 * D, K);
        std::vector<float> x(size_t(D) * KX);
        for (int r = 0; r < D; ++r) {
            for (int k = 0; k < kb; ++k) x[size_t(r) * KX + k] = wx[size_t(r) * kb + k];
            for (int k = 0; k < 2 * W; ++k) x[size_t(r) * KX + kb + k] = wp[size_t(r) * 2 * W + k];
        }
        off[p + "edge_x"] = pk.put(pad_rows(x, D, KX));
        off[p + "edge_xT"] = pk.put(transpose(x, D, KX));
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
        w.edge_x = P(p + "edge_x");
        w.edge_xT = P(p + "edge_xT");
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
    const int NP = 2 * D + H, NG = c.message_groups + 2 * W, KX = c.message_basis_size + 2 * W;
    const int ldx = (KX + 3) & ~3;
    p.N = N;
    p.E = E;
    p.ldrb = (c.message_basis_size + 3) & ~3;
    p.o_gd = ar.add(16 * e);
    p.o_dmom = ar.add(4 * n * m.desc.na * m.desc.nlm);
    p.i_rb = p.add(ar, 4 * e * p.ldrb);
    p.i_fc = p.add(ar, 4 * e);
    p.i_pair = p.add(ar, 4 * e);
    p.i_dv = p.add(ar, 16 * e);
    p.i_harm = p.add(ar, 4 * e * nq);
    p.i_dharm = p.add(ar, 4 * e * nq);
    int dir0 = p.add(ar, 4 * n * CN);
    int x = p.add(ar, 4 * e * ldx);        // shared by the blocks (forward only)
    int eh = p.add(ar, 4 * e * D);         // shared
    for (int b = 0; b < c.message_layers; ++b) {
        BlockBuffers bb;
        bb.h_out = p.add(ar, 4 * n * H);
        bb.rin = p.add(ar, 4 * n);
        bb.vs = p.add(ar, 4 * n * NP);
        bb.ue = p.add(ar, 4 * e * D);
        bb.eh = eh;
        bb.xe = x;
        bb.gv = p.add(ar, 4 * e * NG);
        bb.msg = p.add(ar, 4 * n * H);
        bb.rm = p.add(ar, 4 * n);
        bb.uin = p.add(ar, 4 * n * (H + W));
        bb.u1 = p.add(ar, 4 * n * D);
        bb.z1 = p.add(ar, 4 * n * D);
        bb.dir_in = b == 0 ? dir0 : p.blocks[b - 1].dir_out;
        bb.dir_out = p.add(ar, 4 * n * CN);
        bb.mixstate = p.add(ar, 4 * n * CN);
        p.blocks.push_back(bb);
    }
    p.t_dz1 = p.add(ar, 4 * n * D);
    p.t_duin = p.add(ar, 4 * n * (H + W));
    p.t_dmsg = p.add(ar, 4 * n * H);
    p.t_dvsum = p.add(ar, 4 * n * CN);     // dE/d(dir_out) total
    p.t_dgv = p.add(ar, 4 * e * NG);
    p.t_due = p.add(ar, 4 * e * D);
    p.t_dx = p.add(ar, 4 * e * ldx);
    p.t_dvs = p.add(ar, 4 * n * NP);
    p.t_dmix = p.add(ar, 4 * n * CN);
    p.t_ddir0 = p.add(ar, 4 * n * CN);
    p.t_ddir1 = p.add(ar, 4 * n * CN);
    p.t_dz = p.add(ar, 4 * n * H);
    p.t_dh0 = p.add(ar, 4 * n * H);
    p.t_dh1 = p.add(ar, 4 * n * H);
    p.ldrb_x = ldx;
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
    a.KX = a.kb + 2 * a.lq * a.C;
    a.ldx = p.ldrb_x;
    a.na = m.desc.na;
    a.nlm = m.desc.nlm;
    a.eps = float(c.norm_eps);
    a.cutoff = float(c.message_cutoff);
    a.fc = p.at(p.i_fc);
    a.harm = p.at(p.i_harm);
    a.rb = p.at(p.i_rb);
    a.ldrb = p.ldrb;
    a.node = p.at(bb.vs);
    a.dir_in = p.at(bb.dir_in);
    a.dir_out = p.at(bb.dir_out);
    a.mixw = m.msg[b].mix;
    a.mixst = p.at(bb.mixstate);
    a.x = p.at(bb.xe);
    a.ag = p.at(bb.gv);
    a.msg = p.at(bb.msg);
    a.rm = p.at(bb.rm);
    a.uin = p.at(bb.uin);
    a.duin = p.at(p.t_duin);
    a.dmsg = p.at(p.t_dmsg);
    a.dht = p.at(p.t_dvsum);
    a.dgg = p.at(p.t_dgv);
    a.dv = reinterpret_cast<float4 *>(p.at(p.i_dv));
    a.dy = p.at(p.i_dharm);
    a.dnode = p.at(p.t_dvs);
    a.dmix = p.at(p.t_dmix);
    a.due = p.at(p.t_due);
    a.dx = p.at(p.t_dx);
    return a;
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
    edge_prep(m, p, r, types, s, p.at(p.i_harm), m.harm_scale, lq, nq);
    if (E > 0) RUNE_HIP_CHECK(hipMemsetAsync(p.at(p.i_dharm), 0, 4 * size_t(E) * nq, s));
    hipLaunchKernelGGL(k_eq_encode, dim3(N), dim3(kWave), 0, s, N, moments, m.desc.na,
                       m.desc.nlm, m.enc_w, m.harm_scale, C, nq, p.at(p.blocks[0].dir_in));
    RUNE_HIP_CHECK(hipGetLastError());
    const float *cur = h;
    for (int b = 0; b < c.message_layers; ++b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        EqArgs a = eq_args(m, p, r, b);
        row_inv_rms(N, H, cur, H, float(c.norm_eps), p.at(bb.rin), s);
        Epilogue e0;
        e0.row_scale = p.at(bb.rin);
        gemm(N, w.NP, H, cur, H, w.node_f, H, p.at(bb.vs), w.NP, e0, s);
        hipLaunchKernelGGL(k_eq_mix, dim3(N), dim3(kWave), 0, s, w.mix, p.at(bb.dir_in), C, nq,
                           p.at(bb.mixstate));
        if (E > 0) {
            hipLaunchKernelGGL(k_eq_features, dim3(N), dim3(kWave),
                               sizeof(float) * (2 * C * (nq | 1) + nq), s, a);
            RUNE_HIP_CHECK(hipGetLastError());
            Epilogue e1;
            e1.gtab[0] = p.at(bb.vs);
            e1.gidx[0] = r.ctr;
            e1.gld[0] = w.NP;
            e1.gtab[1] = p.at(bb.vs) + D;
            e1.gidx[1] = r.nbr;
            e1.gld[1] = w.NP;
            e1.gtab[2] = w.pair_proj;
            e1.gidx[2] = reinterpret_cast<const int32_t *>(p.at(p.i_pair));
            e1.gld[2] = D;
            e1.pre = p.at(bb.ue);
            e1.ldp = D;
            e1.act = act;
            gemm(int(E), D, w.KX, p.at(bb.xe), a.ldx, w.edge_x, w.ld_edge_x, p.at(bb.eh), D, e1,
                 s);
            Epilogue e2;
            e2.bias = w.gate_b;
            e2.act = kActSigmoid;
            e2.act_split = c.message_groups;
            e2.act2 = RUNE_ACT_TANH;
            gemm(int(E), w.NG, D, p.at(bb.eh), D, w.gate, D, p.at(bb.gv), w.NG, e2, s);
        }
        hipLaunchKernelGGL(k_eq_aggregate, dim3(N), dim3(kWave),
                           sizeof(float) * (C * nq + w.NG + nq), s, a);
        RUNE_HIP_CHECK(hipGetLastError());
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
    const int CN = C * nq, NU = H + lq * C;
    const int64_t E = p.E;
    float *cur = dh;
    const float *ddir_out = nullptr;   // the last block's states feed only its invariants
    float *ddir_in = p.at(p.t_ddir0);
    for (int b = c.message_layers - 1; b >= 0; --b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        EqArgs a = eq_args(m, p, r, b);
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
        size_t lds = sizeof(float) * (2 * C * (nq | 1) + H + w.NG + nq);
        hipLaunchKernelGGL(k_eq_edge_backward, dim3(N), dim3(kWave), lds, s, a);
        hipLaunchKernelGGL(k_eq_neighbor_backward, dim3(N), dim3(kWave), sizeof(float) * w.NG,
                           s, a);
        RUNE_HIP_CHECK(hipGetLastError());
        if (E > 0) {
            Epilogue e2;
            e2.dact_from = p.at(bb.ue);
            e2.ldu = D;
            e2.dact = act;
            gemm(int(E), D, w.NG, p.at(p.t_dgv), w.NG, w.gate_T, w.NG, p.at(p.t_due), D, e2, s);
            Epilogue e3;
            gemm(int(E), w.KX, D, p.at(p.t_due), D, w.edge_xT, D, p.at(p.t_dx), a.ldx, e3, s);
            edge_rb_backward(m, p, r, p.at(p.t_dx), a.ldx, s);
        }
        const int LC = lq * C;
        hipLaunchKernelGGL(k_eq_atom_backward, dim3(N), dim3(kWave),
                           sizeof(float) * (LC + nq + CN), s, a);
        hipLaunchKernelGGL(k_eq_probe_dy, dim3(N), dim3(kWave),
                           sizeof(float) * (3 * C * (nq | 1) + 3 * LC), s, a);
        RUNE_HIP_CHECK(hipGetLastError());
        Epilogue e4;
        gemm(N, H, w.NP, p.at(p.t_dvs), w.NP, w.node_fT, w.NP, p.at(p.t_dz), H, e4, s);
        float *next = (cur == p.at(p.t_dh0)) ? p.at(p.t_dh1) : p.at(p.t_dh0);
        rms_backward(N, H, p.block_input[b], H, p.at(bb.rin), p.at(p.t_dz), H, cur, H, next, H, s);
        cur = next;
        ddir_out = ddir_in;
        ddir_in = (ddir_in == p.at(p.t_ddir0)) ? p.at(p.t_ddir1) : p.at(p.t_ddir0);
    }
    // ddir_out now holds dE/d(encoder output)
    hipLaunchKernelGGL(k_eq_encoder_backward, dim3(N), dim3(kWave), 0, s, ddir_out, m.enc_w,
                       m.harm_scale, C, nq, m.desc.na, m.desc.nlm, p.dmom);
    if (E > 0) {
        EdgeZ zo;
        for (int k = 0; k < kMaxL + 2; ++k) zo.off[k] = m.desc.z_off[k];
        hipLaunchKernelGGL(k_eq_harmonic_backward, dim3(ceil_div(E, 256)), dim3(256), 0, s, E, r,
                           p.at(p.i_fc), p.at(p.i_dharm), m.desc.z, zo, lq, nq, m.harm_scale,
                           reinterpret_cast<float4 *>(p.at(p.i_dv)));
    }
    RUNE_HIP_CHECK(hipGetLastError());
    edge_direct(p, r, s);
    p.g_direct_used = E > 0;
    p.dmom_used = true;
    return cur;
}

}  // namespace rune
