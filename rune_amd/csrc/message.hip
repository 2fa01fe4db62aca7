// Message blocks.  MP: rune/mobius/message.py:100-193 (grouped scalar messages
// plus the transient l=1 vector branch).  EQ lives in equivariant.hip.
//
// Layout: per-edge tensors are indexed by neighbour record e (see nlist.hpp);
// a record takes part in message passing when it belongs to the radial list
// of its centre, and its cosine cutoff fc(d) (message_cutoff) then weights
// every message term.  Dense maps over atoms or edges are MFMA GEMMs
// (dense.hip); gathers and segment sums are wave-per-atom kernels that walk a
// centre's records (or, for neighbour-destined adjoints, the transpose list)
// in a fixed order, so nothing uses floating-point atomics.
#include <cmath>

#include "activation.hpp"
#include "message.hpp"
#include "wave.hpp"

namespace rune {
namespace {

constexpr int kWave = 64;
constexpr float kPi = 3.14159265358979323846f;
typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ inline float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---- shared edge preparation ----

// One block of 256 threads prepares 256 consecutive records: each thread
// forms its record's rows (masked Chebyshev basis, its distance derivative,
// normalised harmonics) in LDS, then the block writes the tiles out as
// contiguous float4 streams.
__global__ void __launch_bounds__(256) k_edge_prep(EdgePrepArgs a) {
    extern __shared__ float tile[];
    const int ld = a.ldrb, nq = a.harm ? a.nq : 0;
    float *rbL = tile, *rdL = rbL + 256 * ld, *yL = rdL + (a.rbd ? 256 * ld : 0);
    const int64_t e0 = int64_t(blockIdx.x) * 256;
    const int t = threadIdx.x;
    const int64_t e = e0 + t;
    const int rows = int(min<int64_t>(256, a.E - e0));
    if (e < a.E) {
        int i = a.r.ctr[e];
        bool in_r = e >= a.r.view[4 * i] && e < a.r.view[4 * i + 1];
        float4 v = a.r.vec[e];
        float d = v.w;
        float rc = a.cutoff;
        float fc = 0.0f;
        float *rb = rbL + t * ld, *rd = rdL + t * ld;
        for (int k = 0; k < ld; ++k) rb[k] = 0.0f;
        if (a.rbd)
            for (int k = 0; k < ld; ++k) rd[k] = 0.0f;
        if (in_r && d < rc) {
            fc = 0.5f * cosf(kPi * d / rc) + 0.5f;
            const float fp = -0.5f * kPi / rc * sinf(kPi * d / rc);
            const float rs = d / rc - 1.0f;
            const float x = 2.0f * rs * rs - 1.0f, dxdr = 4.0f * rs / rc;
            float half = 0.5f * fc;
            float t2 = 1.0f, t1 = x, u2 = 1.0f, u1 = 2.0f * x;
            rb[0] = 2.0f * half;
            if (a.kb > 1) rb[1] = (x + 1.0f) * half;
            if (a.rbd) {
                rd[0] = fp;
                if (a.kb > 1) rd[1] = 0.5f * dxdr * fc + 0.5f * (x + 1.0f) * fp;
            }
            for (int k = 2; k < a.kb; ++k) {
                float tn = 2.0f * x * t1 - t2;
                float un = 2.0f * x * u1 - u2;
                rb[k] = (tn + 1.0f) * half;
                if (a.rbd) rd[k] = 0.5f * float(k) * u1 * dxdr * fc + 0.5f * (tn + 1.0f) * fp;
                t2 = t1;
                t1 = tn;
                u2 = u1;
                u1 = un;
            }
        }
        a.fc[e] = fc;
        a.pair[e] = a.types[i] * a.n_types + a.types[a.r.nbr[e]];
        a.dv[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (a.dd) a.dd[e] = 0.0f;
        if (a.harm) {
            // normalised real harmonics Y = b(r_hat) * scale (descriptor.py:643-648)
            float *y = yL + t * nq;
            if (!in_r) {
                for (int c = 0; c < nq; ++c) y[c] = 0.0f;
            } else {
                float inv = 1.0f / fmaxf(d, 1.0e-12f);
                harmonics(a.z, a.z_off, a.lq, v.x * inv, v.y * inv, v.z * inv, a.scale, y);
            }
        }
    }
    __syncthreads();
    // ld is a multiple of 4; the harmonic rows are copied as plain floats
    const int n4 = rows * ld / 4;
    for (int q = t; q < n4; q += 256) {
        reinterpret_cast<float4 *>(a.rb + size_t(e0) * ld)[q] = reinterpret_cast<float4 *>(rbL)[q];
        if (a.rbd)
            reinterpret_cast<float4 *>(a.rbd + size_t(e0) * ld)[q] =
                reinterpret_cast<float4 *>(rdL)[q];
    }
    for (int q = t; q < rows * nq; q += 256) a.harm[size_t(e0) * nq + q] = yL[q];
}

// d/dr of the masked Chebyshev basis, accumulated into dv.w:  sum_k drb_k f_k'(d)
__global__ void k_edge_rb_backward(int64_t E, Records r, const float *fc, const float *drb,
                                   int ld, int kb, float cutoff, float4 *dv) {
    int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E || fc[e] == 0.0f) return;
    float d = r.vec[e].w;
    float rc = cutoff;
    float f = 0.5f * cosf(kPi * d / rc) + 0.5f;
    float fp = -0.5f * kPi / rc * sinf(kPi * d / rc);
    float rs = d / rc - 1.0f;
    float x = 2.0f * rs * rs - 1.0f;
    float dxdr = 4.0f * rs / rc;
    const float *g = drb + size_t(e) * ld;
    // k = 0: f0 = fc
    float acc = g[0] * fp;
    float t2 = 1.0f, t1 = x, u2 = 1.0f, u1 = 2.0f * x;
    if (kb > 1) acc += g[1] * (0.5f * dxdr * f + 0.5f * (x + 1.0f) * fp);
    for (int k = 2; k < kb; ++k) {
        float tn = 2.0f * x * t1 - t2;
        float un = 2.0f * x * u1 - u2;
        acc += g[k] * (0.5f * float(k) * u1 * dxdr * f + 0.5f * (tn + 1.0f) * fp);
        t2 = t1;
        t1 = tn;
        u2 = u1;
        u1 = un;
    }
    dv[e].w += acc;
}

// g_direct = dE/dd * u + (I - u u^T) dE/du / d, dE/dd = dv.w (+ dd)
__global__ void k_edge_direct(int64_t E, Records r, const float4 *dv, const float *dd,
                              float4 *g) {
    int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    float4 v = r.vec[e];
    float4 a = dv[e];
    if (dd) a.w += dd[e];
    float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
    float ux = v.x * inv, uy = v.y * inv, uz = v.z * inv;
    float proj = a.x * ux + a.y * uy + a.z * uz;
    g[e] = make_float4(a.w * ux + (a.x - proj * ux) * inv, a.w * uy + (a.y - proj * uy) * inv,
                       a.w * uz + (a.z - proj * uz) * inv, 0.0f);
}

// ---- MP kernels (one 64-lane wave per atom) ----

struct MpArgs {
    Records r;
    int H, G, vc, NG, NP;
    float eps;
    const float *fc;       // [E]
    const float *gv;       // [E, NG] gate logits
    const float *vs;       // [N, NP] values | vector source
    const float *vmix;     // [vc, vc]
    float *msg;            // [N, H]
    float *rm;             // [N]
    float *vsum;           // [N, vc*3]
    float *mixed;          // [N, vc*3]
    float *uin;            // [N, H+vc]
    // reverse
    const float *duin;     // [N, H+vc]
    float *dmsg;           // [N, H]
    float *dvsum;          // [N, vc*3]
    float *dgv;            // [E, NG]
    float4 *dv;            // [E]
    float *dvs;            // [N, NP]
    float cutoff;          // message_cutoff
};

// Lane layout of the MP record loops: a wave walks one atom's records S at a
// time, one record per slot of W = 64 / S lanes; lane sl of a slot owns the
// hidden columns sl, sl + W, sl + 2W, ... (HM of them for H <= 256) and the
// vector channels sl and sl + W.  Record metadata is read 64 records at a
// time lane-parallel and handed to the slots by shuffles; the slots' partial
// sums are folded in a fixed order at the end, so every output has one
// writer and a fixed summation order.
constexpr int kMpSlots = 4, kMpW = kWave / kMpSlots, kMpHM = 256 / kMpW;

// Sigmoid of the group gate of hidden column c (fc folded in).  G <= W: lane
// sl of the slot holds group sl's value and the column reads it by a shuffle
// (executed by every lane); otherwise each column evaluates its own.
__device__ inline float group_gate(float sg, const float *gl, int c, int gw, int G, int slot,
                                   float fc) {
    const float s = bcast(sg, slot * kMpW + min(c / gw, kMpW - 1));
    return G <= kMpW ? s : sigm(gl[c / gw]) * fc;
}

// Scalar and vector messages of centre i (message.py:160-190): msg_i =
// sum_e sig(g_e) fc_e V_j, vsum_i = sum_e sig(v_e) fc_e src_j u_e, then the
// message RMS, the vector mix and its invariants.
__global__ void __launch_bounds__(256) k_mp_aggregate(MpArgs a) {
    __shared__ float vsL[4][64];
    const int i = wave_atom(a.r);
    if (i < 0) return;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
    const int slot = lane / kMpW, sl = lane - slot * kMpW;
    const int H = a.H, G = a.G, vc = a.vc, NG = a.NG, NP = a.NP, gw = H / G;
    float acc[kMpHM], vx[2], vy[2], vz[2];
    zero(acc);
    zero(vx);
    zero(vy);
    zero(vz);
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int b0 = rb; b0 < re; b0 += kWave) {
        const int cnt = min(kWave, re - b0);
        const int ml = min(lane, cnt - 1);
        const float mf = lane < cnt ? a.fc[b0 + ml] : 0.0f;
        const int mj = a.r.nbr[b0 + ml];
        const float4 mv = a.r.vec[b0 + ml];
        for (int q0 = 0; q0 < cnt; q0 += kMpSlots) {
            const int q = min(q0 + slot, cnt - 1);
            const float fq = bcast(mf, q);   // every lane joins the shuffle
            const float fc = q0 + slot < cnt ? fq : 0.0f;
            const int j = bcast(mj, q), e = b0 + q;
            const float *gl = a.gv + size_t(e) * NG;
            const float *vj = a.vs + size_t(j) * NP;
            const float sg = sl < G ? sigm(gl[sl]) * fc : 0.0f;
#pragma unroll
            for (int u = 0; u < kMpHM; ++u) {
                const int c = sl + kMpW * u;
                const float gate = group_gate(sg, gl, min(c, H - 1), gw, G, slot, fc);
                if (c < H) acc[u] += gate * vj[c];
            }
            const float ux = bcast(mv.x, q), uy = bcast(mv.y, q), uz = bcast(mv.z, q);
            const float inv = 1.0f / fmaxf(bcast(mv.w, q), 1.0e-12f);
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int k = sl + kMpW * v;
                if (k < vc) {
                    const float w = sigm(gl[G + k]) * fc * vj[H + k];
                    vx[v] += w * (ux * inv);
                    vy[v] += w * (uy * inv);
                    vz[v] += w * (uz * inv);
                }
            }
        }
    }
    fold_slots<kMpSlots>(acc);
    fold_slots<kMpSlots>(vx);
    fold_slots<kMpSlots>(vy);
    fold_slots<kMpSlots>(vz);
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kMpHM; ++u)
        if (sl + kMpW * u < H) ss += acc[u] * acc[u];
    ss = group_sum(ss, kMpW);
    const float r = 1.0f / sqrtf(ss / float(H) + a.eps);
    const int ldu = H + vc;
    if (slot == 0) {
        if (sl == 0) a.rm[i] = r;
#pragma unroll
        for (int u = 0; u < kMpHM; ++u) {
            const int c = sl + kMpW * u;
            if (c < H) {
                a.msg[size_t(i) * H + c] = acc[u];
                a.uin[size_t(i) * ldu + c] = acc[u] * r;
            }
        }
    }
    if (vc == 0) return;
    float *vs = vsL[wave];
    if (slot == 0) {
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int k = sl + kMpW * v;
            if (k < vc) {
                vs[3 * k] = vx[v];
                vs[3 * k + 1] = vy[v];
                vs[3 * k + 2] = vz[v];
            }
        }
    }
    wave_sync();
    float mx = 0.0f;
    if (lane < 3 * vc) {
        a.vsum[size_t(i) * 3 * vc + lane] = vs[lane];
        const int k = lane / 3, x = lane - 3 * k;
        for (int kk = 0; kk < vc; ++kk) mx += a.vmix[k * vc + kk] * vs[3 * kk + x];
        a.mixed[size_t(i) * 3 * vc + lane] = mx;
    }
    wave_sync();
    if (lane < 3 * vc) vs[lane] = mx;
    wave_sync();
    if (lane < vc) {
        const float t = vs[3 * lane] * vs[3 * lane] + vs[3 * lane + 1] * vs[3 * lane + 1] +
                        vs[3 * lane + 2] * vs[3 * lane + 2];
        a.uin[size_t(i) * ldu + H + lane] = t;
    }
}

__global__ void __launch_bounds__(kWave) k_mp_node_backward(MpArgs a) {
    __shared__ float dmx[3 * 64];
    const int i = blockIdx.x, lane = threadIdx.x;
    const int H = a.H, vc = a.vc, ldu = H + vc;
    const float *d = a.duin + size_t(i) * ldu;
    const float *m = a.msg + size_t(i) * H;
    float dot = 0.0f;
    for (int c = lane; c < H; c += kWave) dot += d[c] * m[c];
    dot = wave_sum(dot);
    float r = a.rm[i];
    float coef = r * r * r * dot / float(H);
    for (int c = lane; c < H; c += kWave) a.dmsg[size_t(i) * H + c] = r * d[c] - coef * m[c];
    if (vc == 0) return;
    if (lane < 3 * vc) {
        int k = lane / 3;
        dmx[lane] = 2.0f * a.mixed[size_t(i) * 3 * vc + lane] * d[H + k];
    }
    __syncthreads();
    if (lane < 3 * vc) {
        int kk = lane / 3, x = lane - 3 * kk;
        float s = 0.0f;
        for (int k = 0; k < vc; ++k) s += a.vmix[k * vc + kk] * dmx[3 * k + x];
        a.dvsum[size_t(i) * 3 * vc + lane] = s;
    }
}

// Adjoint of the gates, fc and the unit vector for the records of centre i
// (slot layout of k_mp_aggregate; the centre's dE/dmsg row and dE/dvsum stay
// in registers).  Group sums P_g = sum_{c in g} dmsg_i[c] V_j[c] go through
// the slot's LDS row.
__global__ void __launch_bounds__(256) k_mp_edge_backward(MpArgs a) {
    extern __shared__ float lds[];
    const int i = wave_atom(a.r);
    if (i < 0) return;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
    const int slot = lane / kMpW, sl = lane - slot * kMpW;
    const int H = a.H, G = a.G, vc = a.vc, NG = a.NG, NP = a.NP, gw = H / G;
    float *pL = lds + (wave * kMpSlots + slot) * (H + 1);   // this slot's products
    float dm[kMpHM], dvx[2], dvy[2], dvz[2];
#pragma unroll
    for (int u = 0; u < kMpHM; ++u) {
        const int c = sl + kMpW * u;
        dm[u] = c < H ? a.dmsg[size_t(i) * H + c] : 0.0f;
    }
    zero(dvx);
    zero(dvy);
    zero(dvz);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const int k = sl + kMpW * v;
        if (k < vc) {
            const float *d = a.dvsum + size_t(i) * 3 * vc + 3 * k;
            dvx[v] = d[0];
            dvy[v] = d[1];
            dvz[v] = d[2];
        }
    }
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int b0 = rb; b0 < re; b0 += kWave) {
        const int cnt = min(kWave, re - b0);
        const int ml = min(lane, cnt - 1);
        const float mf = a.fc[b0 + ml];
        const int mj = a.r.nbr[b0 + ml];
        const float4 mv = a.r.vec[b0 + ml];
        for (int q0 = 0; q0 < cnt; q0 += kMpSlots) {
            const bool live = q0 + slot < cnt;
            const int q = min(q0 + slot, cnt - 1);
            const float fc = bcast(mf, q);
            const int j = bcast(mj, q), e = b0 + q;
            const float4 v = make_float4(bcast(mv.x, q), bcast(mv.y, q), bcast(mv.z, q),
                                         bcast(mv.w, q));
            const float *gl = a.gv + size_t(e) * NG;
            const float *vj = a.vs + size_t(j) * NP;
            const bool on = live && fc != 0.0f;
            if (on) {
#pragma unroll
                for (int u = 0; u < kMpHM; ++u) {
                    const int c = sl + kMpW * u;
                    if (c < H) pL[c] = dm[u] * vj[c];
                }
            }
            wave_sync();
            const float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
            const float u0 = v.x * inv, u1 = v.y * inv, u2 = v.z * inv;
            float contrib = 0.0f, dux = 0.0f, duy = 0.0f, duz = 0.0f;
            float *dg = a.dgv + size_t(e) * NG;
            for (int g = sl; g < G; g += kMpW) {
                float P = 0.0f;
                for (int c = g * gw; c < (g + 1) * gw; ++c) P += pL[c];
                const float sg = sigm(gl[g]);
                if (live) dg[g] = on ? P * fc * sg * (1.0f - sg) : 0.0f;
                contrib += on ? P * sg : 0.0f;
            }
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const int k = sl + kMpW * w;
                if (k < vc) {
                    const float ak = dvx[w] * u0 + dvy[w] * u1 + dvz[w] * u2;
                    const float src = vj[H + k];
                    const float vg = sigm(gl[G + k]);
                    if (live) dg[G + k] = on ? ak * src * fc * vg * (1.0f - vg) : 0.0f;
                    if (on) {
                        contrib += ak * src * vg;
                        const float wt = vg * fc * src;
                        dux += wt * dvx[w];
                        duy += wt * dvy[w];
                        duz += wt * dvz[w];
                    }
                }
            }
            contrib = group_sum(contrib, kMpW);
            dux = group_sum(dux, kMpW);
            duy = group_sum(duy, kMpW);
            duz = group_sum(duz, kMpW);
            if (on && sl == 0) {
                const float fcp = -0.5f * kPi / a.cutoff * sinf(kPi * v.w / a.cutoff);
                float4 acc = a.dv[e];
                acc.x += dux;
                acc.y += duy;
                acc.z += duz;
                acc.w += contrib * fcp;
                a.dv[e] = acc;
            }
            wave_sync();
        }
    }
}

// Adjoint of the gathered neighbour rows (values | vector source) of atom j,
// walking the records whose neighbour is j (slot layout of k_mp_aggregate).
__global__ void __launch_bounds__(256) k_mp_neighbor_backward(MpArgs a) {
    const int j = wave_atom(a.r);
    if (j < 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int slot = lane / kMpW, sl = lane - slot * kMpW;
    const int H = a.H, G = a.G, vc = a.vc, NG = a.NG, NP = a.NP, gw = H / G;
    float acc[kMpHM], av[2];
    zero(acc);
    zero(av);
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    for (int t0 = tb; t0 < te; t0 += kWave) {
        const int cnt = min(kWave, te - t0);
        const int ml = min(lane, cnt - 1);
        const int me = a.r.tidx[t0 + ml];
        const int mi = a.r.tctr[t0 + ml];
        const float mf = lane < cnt ? a.fc[me] : 0.0f;
        const float4 mv = a.r.vec[me];
        for (int q0 = 0; q0 < cnt; q0 += kMpSlots) {
            const int q = min(q0 + slot, cnt - 1);
            const float fq = bcast(mf, q);   // every lane joins the shuffle
            const float fc = q0 + slot < cnt ? fq : 0.0f;
            const int e = bcast(me, q), i = bcast(mi, q);
            const float *gl = a.gv + size_t(e) * NG;
            const float *dmi = a.dmsg + size_t(i) * H;
            const float sg = sl < G ? sigm(gl[sl]) * fc : 0.0f;
#pragma unroll
            for (int u = 0; u < kMpHM; ++u) {
                const int c = sl + kMpW * u;
                const float gate = group_gate(sg, gl, min(c, H - 1), gw, G, slot, fc);
                if (c < H) acc[u] += gate * dmi[c];
            }
            const float inv = 1.0f / fmaxf(bcast(mv.w, q), 1.0e-12f);
            const float vx = bcast(mv.x, q), vy = bcast(mv.y, q), vz = bcast(mv.z, q);
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const int k = sl + kMpW * w;
                if (k < vc) {
                    const float *dvs = a.dvsum + size_t(i) * 3 * vc + 3 * k;
                    const float ak = (dvs[0] * vx + dvs[1] * vy + dvs[2] * vz) * inv;
                    av[w] += sigm(gl[G + k]) * fc * ak;
                }
            }
        }
    }
    fold_slots<kMpSlots>(acc);
    fold_slots<kMpSlots>(av);
    if (slot != 0) return;
#pragma unroll
    for (int u = 0; u < kMpHM; ++u) {
        const int c = sl + kMpW * u;
        if (c < H) a.dvs[size_t(j) * NP + c] = acc[u];
    }
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const int k = sl + kMpW * w;
        if (k < vc) a.dvs[size_t(j) * NP + H + k] = av[w];
    }
}

// ---- MP record kernels, contiguous-column layout ----
// Same slots as above, but lane sl of a slot owns the CH = H / 16 contiguous
// hidden columns sl*CH .. sl*CH + CH - 1, all inside one message group (taken
// when the group width is a multiple of CH, CH divides the rows' 16-byte
// alignment and gw / CH is a power of two): each record then costs a lane one
// gate load and sigmoid and CH/4 vector loads, and the group sums of the
// reverse pass are lane-group sums with no LDS.

template <int CH>
__device__ inline void load_cols(float (&v)[CH], const float *__restrict__ p) {
#pragma unroll
    for (int q = 0; q < CH / 4; ++q) {
        const float4 t = reinterpret_cast<const float4 *>(p)[q];
        v[4 * q] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

template <int CH>
__device__ inline void store_cols(const float (&v)[CH], float *__restrict__ p) {
#pragma unroll
    for (int q = 0; q < CH / 4; ++q)
        reinterpret_cast<float4 *>(p)[q] =
            make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

template <int CH>
__global__ void __launch_bounds__(256) k_mp_aggregate_c(MpArgs a) {
    __shared__ float vsL[4][64];
    const int i = wave_atom(a.r);
    if (i < 0) return;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
    const int slot = lane / kMpW, sl = lane - slot * kMpW;
    const int H = a.H, G = a.G, vc = a.vc, NG = a.NG, NP = a.NP, gw = H / G;
    const int c0 = sl * CH, g = c0 / gw;
    float acc[CH], vx[2], vy[2], vz[2];
    zero(acc);
    zero(vx);
    zero(vy);
    zero(vz);
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int b0 = rb; b0 < re; b0 += kWave) {
        const int cnt = min(kWave, re - b0);
        const int ml = min(lane, cnt - 1);
        const float mf = lane < cnt ? a.fc[b0 + ml] : 0.0f;
        const int mj = a.r.nbr[b0 + ml];
        const float4 mv = a.r.vec[b0 + ml];
#pragma unroll 2
        for (int q0 = 0; q0 < cnt; q0 += kMpSlots) {
            const int q = min(q0 + slot, cnt - 1);
            const float fq = bcast(mf, q);   // every lane joins the shuffle
            const float fc = q0 + slot < cnt ? fq : 0.0f;
            const int j = bcast(mj, q), e = b0 + q;
            const float *gl = a.gv + size_t(e) * NG;
            const float *vj = a.vs + size_t(j) * NP;
            float val[CH];
            load_cols(val, vj + c0);
            const float sg = sigm(gl[g]) * fc;
#pragma unroll
            for (int t = 0; t < CH; ++t) acc[t] += sg * val[t];
            const float ux = bcast(mv.x, q), uy = bcast(mv.y, q), uz = bcast(mv.z, q);
            const float inv = 1.0f / fmaxf(bcast(mv.w, q), 1.0e-12f);
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int k = sl + kMpW * v;
                if (k < vc) {
                    const float w = sigm(gl[G + k]) * fc * vj[H + k];
                    vx[v] += w * (ux * inv);
                    vy[v] += w * (uy * inv);
                    vz[v] += w * (uz * inv);
                }
            }
        }
    }
    fold_slots<kMpSlots>(acc);
    fold_slots<kMpSlots>(vx);
    fold_slots<kMpSlots>(vy);
    fold_slots<kMpSlots>(vz);
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < CH; ++t) ss += acc[t] * acc[t];
    ss = group_sum(ss, kMpW);
    const float r = 1.0f / sqrtf(ss / float(H) + a.eps);
    const int ldu = H + vc;
    if (slot == 0) {
        if (sl == 0) a.rm[i] = r;
        store_cols(acc, a.msg + size_t(i) * H + c0);
#pragma unroll
        for (int t = 0; t < CH; ++t) a.uin[size_t(i) * ldu + c0 + t] = acc[t] * r;
    }
    if (vc == 0) return;
    float *vs = vsL[wave];
    if (slot == 0) {
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int k = sl + kMpW * v;
            if (k < vc) {
                vs[3 * k] = vx[v];
                vs[3 * k + 1] = vy[v];
                vs[3 * k + 2] = vz[v];
            }
        }
    }
    wave_sync();
    float mx = 0.0f;
    if (lane < 3 * vc) {
        a.vsum[size_t(i) * 3 * vc + lane] = vs[lane];
        const int k = lane / 3, x = lane - 3 * k;
        for (int kk = 0; kk < vc; ++kk) mx += a.vmix[k * vc + kk] * vs[3 * kk + x];
        a.mixed[size_t(i) * 3 * vc + lane] = mx;
    }
    wave_sync();
    if (lane < 3 * vc) vs[lane] = mx;
    wave_sync();
    if (lane < vc) {
        const float t = vs[3 * lane] * vs[3 * lane] + vs[3 * lane + 1] * vs[3 * lane + 1] +
                        vs[3 * lane + 2] * vs[3 * lane + 2];
        a.uin[size_t(i) * ldu + H + lane] = t;
    }
}

// 8 waves per SIMD (five registers spill) measured faster on C3 than the
// unbounded 6.
template <int CH>
__global__ void __launch_bounds__(256, 8) k_mp_edge_backward_c(MpArgs a) {
    const int i = wave_atom(a.r);
    if (i < 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int slot = lane / kMpW, sl = lane - slot * kMpW;
    const int H = a.H, G = a.G, vc = a.vc, NG = a.NG, NP = a.NP, gw = H / G;
    const int c0 = sl * CH, g = c0 / gw, lg = gw / CH;   // lg lanes per group
    const bool lead = sl % lg == 0;
    float dm[CH], dvx[2], dvy[2], dvz[2];
    load_cols(dm, a.dmsg + size_t(i) * H + c0);
    zero(dvx);
    zero(dvy);
    zero(dvz);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const int k = sl + kMpW * v;
        if (k < vc) {
            const float *d = a.dvsum + size_t(i) * 3 * vc + 3 * k;
            dvx[v] = d[0];
            dvy[v] = d[1];
            dvz[v] = d[2];
        }
    }
    const int rb = a.r.view[4 * i], re = a.r.view[4 * i + 1];
    for (int b0 = rb; b0 < re; b0 += kWave) {
        const int cnt = min(kWave, re - b0);
        const int ml = min(lane, cnt - 1);
        const float mf = a.fc[b0 + ml];
        const int mj = a.r.nbr[b0 + ml];
        const float4 mv = a.r.vec[b0 + ml];
#pragma unroll 2
        for (int q0 = 0; q0 < cnt; q0 += kMpSlots) {
            const bool live = q0 + slot < cnt;
            const int q = min(q0 + slot, cnt - 1);
            const float fc = bcast(mf, q);
            const int j = bcast(mj, q), e = b0 + q;
            const float4 v = make_float4(bcast(mv.x, q), bcast(mv.y, q), bcast(mv.z, q),
                                         bcast(mv.w, q));
            const float *gl = a.gv + size_t(e) * NG;
            const float *vj = a.vs + size_t(j) * NP;
            const bool on = live && fc != 0.0f;
            float val[CH];
            load_cols(val, vj + c0);
            float P = 0.0f;
#pragma unroll
            for (int t = 0; t < CH; ++t) P += dm[t] * val[t];
            P = group_sum(P, lg);
            const float sg = sigm(gl[g]);
            float *dg = a.dgv + size_t(e) * NG;
            if (live && lead) dg[g] = on ? P * fc * sg * (1.0f - sg) : 0.0f;
            float contrib = on && lead ? P * sg : 0.0f;
            const float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
            const float u0 = v.x * inv, u1 = v.y * inv, u2 = v.z * inv;
            float dux = 0.0f, duy = 0.0f, duz = 0.0f;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const int k = sl + kMpW * w;
                if (k < vc) {
                    const float ak = dvx[w] * u0 + dvy[w] * u1 + dvz[w] * u2;
                    const float src = vj[H + k];
                    const float vg = sigm(gl[G + k]);
                    if (live) dg[G + k] = on ? ak * src * fc * vg * (1.0f - vg) : 0.0f;
                    if (on) {
                        contrib += ak * src * vg;
                        const float wt = vg * fc * src;
                        dux += wt * dvx[w];
                        duy += wt * dvy[w];
                        duz += wt * dvz[w];
                    }
                }
            }
            contrib = group_sum(contrib, kMpW);
            dux = group_sum(dux, kMpW);
            duy = group_sum(duy, kMpW);
            duz = group_sum(duz, kMpW);
            if (on && sl == 0) {
                const float fcp = -0.5f * kPi / a.cutoff * sinf(kPi * v.w / a.cutoff);
                float4 acc = a.dv[e];
                acc.x += dux;
                acc.y += duy;
                acc.z += duz;
                acc.w += contrib * fcp;
                a.dv[e] = acc;
            }
        }
    }
}

template <int CH>
__global__ void __launch_bounds__(256) k_mp_neighbor_backward_c(MpArgs a) {
    const int j = wave_atom(a.r);
    if (j < 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int slot = lane / kMpW, sl = lane - slot * kMpW;
    const int H = a.H, G = a.G, vc = a.vc, NG = a.NG, NP = a.NP, gw = H / G;
    const int c0 = sl * CH, g = c0 / gw;
    float acc[CH], av[2];
    zero(acc);
    zero(av);
    const int tb = a.r.tptr[j], te = a.r.tptr[j + 1];
    for (int t0 = tb; t0 < te; t0 += kWave) {
        const int cnt = min(kWave, te - t0);
        const int ml = min(lane, cnt - 1);
        const int me = a.r.tidx[t0 + ml];
        const int mi = a.r.tctr[t0 + ml];
        const float mf = lane < cnt ? a.fc[me] : 0.0f;
        const float4 mv = a.r.vec[me];
#pragma unroll 2
        for (int q0 = 0; q0 < cnt; q0 += kMpSlots) {
            const int q = min(q0 + slot, cnt - 1);
            const float fq = bcast(mf, q);   // every lane joins the shuffle
            const float fc = q0 + slot < cnt ? fq : 0.0f;
            const int e = bcast(me, q), i = bcast(mi, q);
            const float *gl = a.gv + size_t(e) * NG;
            float dmi[CH];
            load_cols(dmi, a.dmsg + size_t(i) * H + c0);
            const float sg = sigm(gl[g]) * fc;
#pragma unroll
            for (int t = 0; t < CH; ++t) acc[t] += sg * dmi[t];
            const float inv = 1.0f / fmaxf(bcast(mv.w, q), 1.0e-12f);
            const float vx = bcast(mv.x, q), vy = bcast(mv.y, q), vz = bcast(mv.z, q);
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const int k = sl + kMpW * w;
                if (k < vc) {
                    const float *dvs = a.dvsum + size_t(i) * 3 * vc + 3 * k;
                    const float ak = (dvs[0] * vx + dvs[1] * vy + dvs[2] * vz) * inv;
                    av[w] += sigm(gl[G + k]) * fc * ak;
                }
            }
        }
    }
    fold_slots<kMpSlots>(acc);
    fold_slots<kMpSlots>(av);
    if (slot != 0) return;
    store_cols(acc, a.dvs + size_t(j) * NP + c0);
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const int k = sl + kMpW * w;
        if (k < vc) a.dvs[size_t(j) * NP + H + k] = av[w];
    }
}

// ---- MP edge MLP on the matrix cores, nothing per record but the gates ----
// Forward, per 16-record tile and wave: u^T = W_rb rb^T + pair row (edge_mlp.0
// with its bias folded into the pair table), h = act(u), gate logits
// g^T = W_g h^T + b (message.py:108-111, :160, :178).  Reverse: u is formed
// again, due^T = (W_g^T dgv^T) * act'(u^T) and drb^T = W_rb^T due^T.  With
// v_mfma_f32_16x16x4f32 (lane l supplies A[l%16][k], B[k][l%16] for the k
// its lane group l/16 feeds; accumulator v of lane l is C[4(l/16)+v][l%16])
// the transposed products keep record r = l%16 in every lane's columns, so
// the accumulator of one product is the B operand of the next (dimension
// d = 16q + 4(l/16) + v of record r) and u, h and due never leave
// registers.  Weights sit in LDS for the whole launch; waves stride over
// the tiles.  This replaces the [E, D] pre-activation array and the three
// per-record GEMMs that wrote and read it.
struct MpEdgeArgs {
    int64_t E;
    const float *rb;       // [E, ldrb]
    int ldrb, kb, KP;      // basis size, row stride of W_rb (= kb rounded to 4)
    const int32_t *pair;   // [E]
    const float *Wx;       // [D, KP]  edge_mlp.0 radial columns
    const float *P;        // [T*T, D] pair rows (+ bias)
    const float *Wg;       // [NG, D]  gate rows
    const float *gb;       // [NG]
    int D, NG, act;
    float *gv;             // forward out [E, NG]
    const float *dgv;      // reverse in  [E, NG]
    float *drb;            // reverse out [E, ldrb], or null when dv takes its contraction
    const float *fc;       // [E] cosine cutoff (0: record outside the message list)
    const float4 *vec;     // [E] record vectors
    float4 *dv;            // [E] dE/dd accumulated in .w (dv.w += sum_k drb_k f_k'(d))
    float *dd;             // [E] or null: the accumulator of that sum instead of dv.w
    float cutoff;          // message_cutoff
};

// Operands of one tile that come from memory, loaded one tile ahead: the
// radial basis values this lane feeds (k = 4s + g) and the record's pair.
constexpr int kMpKS = 8;   // KP <= 32
struct MpTileIn {
    float rb[kMpKS];
    int pair;
};

__device__ inline void mp_tile_load(const MpEdgeArgs &a, int64_t e, int g, MpTileIn &in) {
    const float *rbr = a.rb + size_t(e) * a.ldrb;
#pragma unroll
    for (int s = 0; s < kMpKS; ++s) in.rb[s] = 4 * s < a.KP ? rbr[4 * s + g] : 0.0f;
    in.pair = a.pair[e];
}

// u^T of one tile: acc[q][v] = u[r][16q + 4g + v] (pair row and bias added).
template <int DB>
__device__ inline void mp_edge_u(const MpEdgeArgs &a, const float *Wx, const MpTileIn &in, int r,
                                 int g, float (&acc)[DB][4]) {
    const float *pr = a.P + size_t(in.pair) * a.D + 4 * g;
    float4 pv[DB];
#pragma unroll
    for (int q = 0; q < DB; ++q) pv[q] = *reinterpret_cast<const float4 *>(pr + 16 * q);
    floatx4_t m[DB];
#pragma unroll
    for (int q = 0; q < DB; ++q) m[q] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // k-step s feeds k = 4s + g from every lane group
#pragma unroll
    for (int s = 0; s < kMpKS; ++s) {
        if (4 * s >= a.KP) break;
#pragma unroll
        for (int q = 0; q < DB; ++q)
            m[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(Wx[(16 * q + r) * a.KP + 4 * s + g],
                                                        in.rb[s], m[q], 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < DB; ++q) {
        acc[q][0] = m[q][0] + pv[q].x;
        acc[q][1] = m[q][1] + pv[q].y;
        acc[q][2] = m[q][2] + pv[q].z;
        acc[q][3] = m[q][3] + pv[q].w;
    }
}

// Register budgets measured on C3: the forward at 4 waves per SIMD (no
// spill) and the reverse at 3 (four spilled registers) beat the compiler's
// unbounded choices (3 and 2 waves); the reverse at 4 spills 60 and loses.
template <int DB, int GB, int ACT>
__global__ void __launch_bounds__(256, 4) k_mp_edge_forward(MpEdgeArgs a) {
    extern __shared__ float lds[];
    float *Wx = lds;                      // [D][KP]
    float *Wg = Wx + a.D * a.KP;          // [16 GB][D], zero rows past NG
    for (int o = threadIdx.x; o < a.D * a.KP; o += 256) Wx[o] = a.Wx[o];
    for (int o = threadIdx.x; o < 16 * GB * a.D; o += 256)
        Wg[o] = o < a.NG * a.D ? a.Wg[o] : 0.0f;
    __syncthreads();
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int64_t tiles = (a.E + 15) / 16;
    const int64_t waves = int64_t(gridDim.x) * 4;
    int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    MpTileIn in;
    if (t < tiles) mp_tile_load(a, min(16 * t + r, a.E - 1), g, in);
    for (; t < tiles; t += waves) {
        const int64_t e = min(16 * t + r, a.E - 1);
        float u[DB][4];
        mp_edge_u<DB>(a, Wx, in, r, g, u);
        if (t + waves < tiles) mp_tile_load(a, min(16 * (t + waves) + r, a.E - 1), g, in);
#pragma unroll
        for (int q = 0; q < DB; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v) u[q][v] = act_f(ACT, u[q][v]);
        // g^T[16 gb + 4g + v][r]: k-step (q, v) feeds d = 16q + 4g + v
#pragma unroll
        for (int b = 0; b < GB; ++b) {
            floatx4_t m = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const float *wr = Wg + (16 * b + r) * a.D + 4 * g;
#pragma unroll
            for (int q = 0; q < DB; ++q) {
                const float4 w = *reinterpret_cast<const float4 *>(wr + 16 * q);
                m = __builtin_amdgcn_mfma_f32_16x16x4f32(w.x, u[q][0], m, 0, 0, 0);
                m = __builtin_amdgcn_mfma_f32_16x16x4f32(w.y, u[q][1], m, 0, 0, 0);
                m = __builtin_amdgcn_mfma_f32_16x16x4f32(w.z, u[q][2], m, 0, 0, 0);
                m = __builtin_amdgcn_mfma_f32_16x16x4f32(w.w, u[q][3], m, 0, 0, 0);
            }
            if (16 * t + r < a.E) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int o = 16 * b + 4 * g + v;
                    if (o < a.NG) a.gv[size_t(e) * a.NG + o] = m[v] + a.gb[o];
                }
            }
        }
    }
}

template <int DB, int GB, int ACT>
__global__ void __launch_bounds__(256, 3) k_mp_edge_reverse(MpEdgeArgs a) {
    extern __shared__ float lds[];
    float *Wx = lds;                      // [D][KP]
    float *WgT = Wx + a.D * a.KP;         // [D][16 GB], zero columns past NG
    const int ng16 = 16 * GB;
    for (int o = threadIdx.x; o < a.D * a.KP; o += 256) Wx[o] = a.Wx[o];
    for (int o = threadIdx.x; o < a.D * ng16; o += 256) {
        const int d = o / ng16, k = o - d * ng16;
        WgT[o] = k < a.NG ? a.Wg[size_t(k) * a.D + d] : 0.0f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int64_t tiles = (a.E + 15) / 16;
    const int64_t waves = int64_t(gridDim.x) * 4;
    const int KBF = a.kb / 16, tail = a.kb - 16 * KBF;   // MFMA rows of drb, VALU rows
    int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    MpTileIn in;
    float dgn[GB][4];
    auto load_dg = [&](int64_t e) {
        const float *dg = a.dgv + size_t(e) * a.NG;
#pragma unroll
        for (int b = 0; b < GB; ++b)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int o = 16 * b + 4 * s + g;
                dgn[b][s] = o < a.NG ? dg[o] : 0.0f;
            }
    };
    if (t < tiles) {
        mp_tile_load(a, min(16 * t + r, a.E - 1), g, in);
        load_dg(min(16 * t + r, a.E - 1));
    }
    for (; t < tiles; t += waves) {
        const int64_t e = min(16 * t + r, a.E - 1);
        float u[DB][4];
        mp_edge_u<DB>(a, Wx, in, r, g, u);
        float dgc[GB][4];
#pragma unroll
        for (int b = 0; b < GB; ++b)
#pragma unroll
            for (int s = 0; s < 4; ++s) dgc[b][s] = dgn[b][s];
        if (t + waves < tiles) {
            const int64_t en = min(16 * (t + waves) + r, a.E - 1);
            mp_tile_load(a, en, g, in);
            load_dg(en);
        }
        // due^T[d][r] = sum_o W_g[o][d] dgv[r][o]: k-step s of block b feeds
        // o = 16b + 4s + g
        floatx4_t m[DB];
#pragma unroll
        for (int q = 0; q < DB; ++q) m[q] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < GB; ++b)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int o = 16 * b + 4 * s + g;
#pragma unroll
                for (int q = 0; q < DB; ++q)
                    m[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(WgT[(16 * q + r) * ng16 + o],
                                                                dgc[b][s], m[q], 0, 0, 0);
            }
#pragma unroll
        for (int q = 0; q < DB; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v) u[q][v] = m[q][v] * act_d(ACT, u[q][v]);   // due
        const bool live = 16 * t + r < a.E;
        // drb^T[16p + 4g + v][r] = sum_d W_rb[d][k] due^T[d][r] for the full
        // 16-row blocks (k-step (q, v), two accumulators), then the last
        // kb % 16 rows as lane dot products summed over the four lane groups
        float w[2][4];
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
            floatx4_t acc0 = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
            if (pb < KBF) {
                const int k = 16 * pb + r;
#pragma unroll
                for (int q = 0; q < DB; ++q)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float wa = Wx[(16 * q + 4 * g + v) * a.KP + k];
                        if (q & 1)
                            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(wa, u[q][v], acc1, 0, 0, 0);
                        else
                            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(wa, u[q][v], acc0, 0, 0, 0);
                    }
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) w[pb][v] = acc0[v] + acc1[v];
        }
        float wt[4];   // tail rows k = 16 KBF + j, this lane's share over its d
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float sum = 0.0f;
            if (j < tail) {
#pragma unroll
                for (int q = 0; q < DB; ++q)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        sum += Wx[(16 * q + 4 * g + v) * a.KP + 16 * KBF + j] * u[q][v];
            }
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            wt[j] = sum;
        }
        if (!a.dv) {
            if (live) {
#pragma unroll
                for (int pb = 0; pb < 2; ++pb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (pb < KBF) a.drb[size_t(e) * a.ldrb + 16 * pb + 4 * g + v] = w[pb][v];
                if (g == 0)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (j < tail) a.drb[size_t(e) * a.ldrb + 16 * KBF + j] = wt[j];
            }
            continue;
        }
        // dE/dd += sum_k drb_k f_k'(d) (masked Chebyshev basis, message.py:108-110):
        // each lane group adds its own k of the full blocks, lane group 0 the
        // tail rows, then the four groups of record r are summed
        const float d = a.vec[e].w, rc = a.cutoff;
        const float f = 0.5f * cosf(kPi * d / rc) + 0.5f;
        const float fp = -0.5f * kPi / rc * sinf(kPi * d / rc);
        const float rs = d / rc - 1.0f;
        const float x = 2.0f * rs * rs - 1.0f, dxdr = 4.0f * rs / rc;
        float t2 = 1.0f, t1 = x, u2 = 1.0f, u1 = 2.0f * x;
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < 36; ++k) {   // 2 full blocks + 4 tail rows
            if (k >= a.kb) continue;
            float dk;
            if (k == 0) {
                dk = fp;
            } else if (k == 1) {
                dk = 0.5f * dxdr * f + 0.5f * (x + 1.0f) * fp;
            } else {
                const float tn = 2.0f * x * t1 - t2, un = 2.0f * x * u1 - u2;
                dk = 0.5f * float(k) * u1 * dxdr * f + 0.5f * (tn + 1.0f) * fp;
                t2 = t1;
                t1 = tn;
                u2 = u1;
                u1 = un;
            }
            if (k < 32) {
                const int pb = k >> 4;
                if (pb < KBF && ((k >> 2) & 3) == g) part += w[pb][k & 3] * dk;
            }
            if (k >= 16 * KBF && k < 16 * KBF + 4 && g == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (k == 16 * KBF + j) part += wt[j] * dk;
            }
        }
        part += __shfl_xor(part, 16, 64);
        part += __shfl_xor(part, 32, 64);
        if (live && g == 0 && a.fc[e] != 0.0f) {
            if (a.dd)
                a.dd[e] += part;
            else
                a.dv[e].w += part;
        }
    }
}

// Columns per lane of the contiguous-column kernels for this model, or 0 when
// the strided kernels are used.
int mp_columns(int H, int G, int NP) {
    if (H != 64 && H != 128 && H != 256) return 0;
    const int ch = H / kMpW, gw = H / G;
    if (gw % ch != 0 || NP % 4 != 0) return 0;
    const int lg = gw / ch;
    return (lg & (lg - 1)) == 0 ? ch : 0;
}

// Launch of the fused MP edge MLP (forward or reverse), or false when the
// model's widths have no instantiation (the per-record GEMMs are used then).
// Widths the fused kernels are instantiated for: D in {32, 64, 96, 128},
// at most 32 gates, basis rows padded to at most 32 and at most four rows past
// the last full 16-row block of drb.
bool mp_edge_fusable(int D, int NG, int kb) {
    const int DB = D / 16, KP = (kb + 3) & ~3;
    return D % 16 == 0 && (DB == 2 || DB == 4 || DB == 6 || DB == 8) && NG <= 32 && KP <= 32 &&
           kb - 16 * (kb / 16) <= 4;
}

bool mp_edge_fused(const MpEdgeArgs &a, bool reverse, hipStream_t s) {
    const int DB = a.D / 16, GB = (a.NG + 15) / 16;
    if (!mp_edge_fusable(a.D, a.NG, a.kb)) return false;
    if (a.E == 0) return true;
    const size_t lds = sizeof(float) * (size_t(a.D) * a.KP + size_t(16) * GB * a.D);
    const int64_t tiles = (a.E + 15) / 16;
    const dim3 grid(unsigned(std::min<int64_t>((tiles + 3) / 4, 2048))), block(256);
#define MP_EDGE_ACT(K, D_, G_, A_)                                                   \
    if (DB == D_ && GB == G_ && a.act == A_) {                                       \
        hipLaunchKernelGGL((K<D_, G_, A_>), grid, block, lds, s, a);                 \
        return true;                                                                 \
    }
#define MP_EDGE(K, D_, G_)                                                           \
    MP_EDGE_ACT(K, D_, G_, RUNE_ACT_TANH)                                            \
    MP_EDGE_ACT(K, D_, G_, RUNE_ACT_SILU) MP_EDGE_ACT(K, D_, G_, RUNE_ACT_GELU)
#define MP_EDGE_ALL(K)                                                               \
    MP_EDGE(K, 2, 1) MP_EDGE(K, 4, 1) MP_EDGE(K, 6, 1) MP_EDGE(K, 8, 1)              \
    MP_EDGE(K, 2, 2) MP_EDGE(K, 4, 2) MP_EDGE(K, 6, 2) MP_EDGE(K, 8, 2)
    if (reverse) {
        MP_EDGE_ALL(k_mp_edge_reverse)
    } else {
        MP_EDGE_ALL(k_mp_edge_forward)
    }
#undef MP_EDGE_ALL
#undef MP_EDGE
#undef MP_EDGE_ACT
    return false;
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

void MessagePlan::bind(char *base) {
    ptrs.clear();
    for (size_t o : offs) ptrs.push_back(reinterpret_cast<float *>(base + o));
    if (o_gd || o_dmom) {
        g_direct = reinterpret_cast<float4 *>(base + o_gd);
        dmom = reinterpret_cast<float *>(base + o_dmom);
    }
}

void validate_messages(ModelImpl &m) {
    const rune_model_config &c = m.cfg;
    if (c.family != RUNE_FAMILY_MOBIUS || c.message_layers == 0) return;
    RUNE_REQUIRE(c.hidden_dim <= 256, RUNE_ERR_ARGUMENT,
                 "message blocks support hidden_dim <= 256");
    RUNE_REQUIRE(c.message_groups >= 1 && c.hidden_dim % c.message_groups == 0,
                 RUNE_ERR_ARGUMENT, "hidden_dim must be divisible by message_groups.");
    RUNE_REQUIRE(c.message_basis_size >= 1 && c.message_basis_size <= 64, RUNE_ERR_ARGUMENT,
                 "message_basis_size outside [1, 64]");
    RUNE_REQUIRE(c.message_cutoff > 0 && c.message_cutoff <= c.rc_radial, RUNE_ERR_ARGUMENT,
                 "message_cutoff must be positive and cannot exceed rcut_radial.");
    if (c.message_mode == RUNE_MESSAGE_SCALAR) {
        RUNE_REQUIRE(c.vector_channels <= 21, RUNE_ERR_ARGUMENT,
                     "vector_channels outside [0, 21]");
        RUNE_REQUIRE(c.message_groups + c.vector_channels <= kWave, RUNE_ERR_ARGUMENT,
                     "message_groups + vector_channels must not exceed 64");
    } else {
        validate_equivariant(m);
    }
}

static void expect(ModelImpl &m, const std::string &name, int64_t n) { m.expected[name] = n; }

void define_expected_messages(ModelImpl &m) {
    const rune_model_config &c = m.cfg;
    const int64_t T = c.n_types, H = c.hidden_dim, D = c.message_dim, P = c.pair_dim;
    const int64_t G = c.message_groups, vc = c.vector_channels, kb = c.message_basis_size;
    if (c.message_mode == RUNE_MESSAGE_EQUIVARIANT) {
        define_expected_equivariant(m);
        return;
    }
    for (int b = 0; b < c.message_layers; ++b) {
        std::string p = "message_blocks." + std::to_string(b) + ".";
        expect(m, p + "input_norm.weight", H);
        expect(m, p + "pair_embedding.weight", T * T * P);
        expect(m, p + "edge_mlp.0.weight", D * (kb + P));
        expect(m, p + "edge_mlp.0.bias", D);
        expect(m, p + "group_gate.weight", G * D);
        expect(m, p + "group_gate.bias", G);
        expect(m, p + "value_projection.weight", H * H);
        if (vc) {
            expect(m, p + "vector_gate.weight", vc * D);
            expect(m, p + "vector_gate.bias", vc);
            expect(m, p + "vector_source.weight", vc * H);
            expect(m, p + "vector_mix.weight", vc * vc);
        }
        expect(m, p + "message_norm.weight", H);
        expect(m, p + "update.0.weight", D * (H + vc));
        expect(m, p + "update.0.bias", D);
        expect(m, p + "update.2.weight", H * D);
        expect(m, p + "update.2.bias", H);
    }
}

// rows [r0, r1) of W [rows, cols] scaled column-wise by s (s may be null)
std::vector<float> fold_cols(const std::vector<float> &w, int rows, int cols, const float *s) {
    std::vector<float> out(w.begin(), w.begin() + size_t(rows) * cols);
    if (s)
        for (int r = 0; r < rows; ++r)
            for (int c = 0; c < cols; ++c) out[size_t(r) * cols + c] *= s[c];
    return out;
}

std::vector<float> columns(const std::vector<float> &w, int rows, int cols, int c0, int c1) {
    std::vector<float> out(size_t(rows) * (c1 - c0));
    for (int r = 0; r < rows; ++r)
        for (int c = c0; c < c1; ++c) out[size_t(r) * (c1 - c0) + c - c0] = w[size_t(r) * cols + c];
    return out;
}

// pair_embedding [T*T, P] x W[:, c0:c0+P]^T + b  -> [T*T, D]
std::vector<float> pair_projection(const std::vector<float> &emb, const std::vector<float> &w,
                                   const std::vector<float> &b, int TT, int P, int D, int K,
                                   int c0) {
    std::vector<float> out(size_t(TT) * D);
    for (int t = 0; t < TT; ++t)
        for (int o = 0; o < D; ++o) {
            double acc = 0.0;
            for (int p = 0; p < P; ++p)
                acc += double(emb[size_t(t) * P + p]) * double(w[size_t(o) * K + c0 + p]);
            out[size_t(t) * D + o] = float(acc + double(b[o]));
        }
    return out;
}

void pack_messages(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off) {
    const rune_model_config &c = m.cfg;
    if (c.message_layers == 0) return;
    if (c.message_mode == RUNE_MESSAGE_EQUIVARIANT) {
        pack_equivariant(m, pk, off);
        return;
    }
    const int T = c.n_types, H = c.hidden_dim, D = c.message_dim, P = c.pair_dim;
    const int G = c.message_groups, vc = c.vector_channels, kb = c.message_basis_size;
    const int NP = H + vc, NG = G + vc, K = kb + P;
    for (int b = 0; b < c.message_layers; ++b) {
        std::string p = "message_blocks." + std::to_string(b) + ".";
        const auto &win = m.tensor(p + "input_norm.weight");
        std::vector<float> node = m.tensor(p + "value_projection.weight");   // [H, H]
        if (vc) {
            const auto &src = m.tensor(p + "vector_source.weight");           // [vc, H]
            node.insert(node.end(), src.begin(), src.end());
        }
        node = fold_cols(node, NP, H, win.data());
        off[p + "node_f"] = pk.put(node);
        off[p + "node_fT"] = pk.put(transpose(node, NP, H));
        const auto &we = m.tensor(p + "edge_mlp.0.weight");                   // [D, K]
        std::vector<float> wx = columns(we, D, K, 0, kb);
        off[p + "edge_x"] = pk.put(pad_rows(wx, D, kb));
        off[p + "edge_xT"] = pk.put(transpose(wx, D, kb));
        off[p + "pair_proj"] = pk.put(pair_projection(m.tensor(p + "pair_embedding.weight"), we,
                                                      m.tensor(p + "edge_mlp.0.bias"), T * T, P,
                                                      D, K, kb));
        std::vector<float> gate = m.tensor(p + "group_gate.weight");         // [G, D]
        std::vector<float> gb = m.tensor(p + "group_gate.bias");
        if (vc) {
            const auto &vg = m.tensor(p + "vector_gate.weight");
            gate.insert(gate.end(), vg.begin(), vg.end());
            const auto &vb = m.tensor(p + "vector_gate.bias");
            gb.insert(gb.end(), vb.begin(), vb.end());
            off[p + "vmix"] = pk.put(m.tensor(p + "vector_mix.weight"));
        }
        off[p + "gate"] = pk.put(gate);
        off[p + "gate_T"] = pk.put(transpose(gate, NG, D));
        off[p + "gate_b"] = pk.put(gb);
        std::vector<float> wmsg = m.tensor(p + "message_norm.weight");
        wmsg.resize(NP, 1.0f);                                                 // invariants unscaled
        std::vector<float> up1 = fold_cols(m.tensor(p + "update.0.weight"), D, NP, wmsg.data());
        off[p + "up1_f"] = pk.put(up1);
        off[p + "up1_fT"] = pk.put(transpose(up1, D, NP));
        off[p + "up1_b"] = pk.put(m.tensor(p + "update.0.bias"));
        const auto &up2 = m.tensor(p + "update.2.weight");                    // [H, D]
        off[p + "up2"] = pk.put(up2);
        off[p + "up2_T"] = pk.put(transpose(up2, H, D));
        off[p + "up2_b"] = pk.put(m.tensor(p + "update.2.bias"));
    }
}

void bind_messages(ModelImpl &m, const PackedLookup &P) {
    const rune_model_config &c = m.cfg;
    if (c.message_layers == 0) return;
    if (c.message_mode == RUNE_MESSAGE_EQUIVARIANT) {
        bind_equivariant(m, P);
        return;
    }
    m.msg.resize(c.message_layers);
    for (int b = 0; b < c.message_layers; ++b) {
        std::string p = "message_blocks." + std::to_string(b) + ".";
        MessageWeights &w = m.msg[b];
        w.NP = c.hidden_dim + c.vector_channels;
        w.NG = c.message_groups + c.vector_channels;
        w.KX = c.message_basis_size;
        w.ld_edge_x = (w.KX + 3) & ~3;
        w.node_f = P(p + "node_f");
        w.node_fT = P(p + "node_fT");
        w.edge_x = P(p + "edge_x");
        w.edge_xT = P(p + "edge_xT");
        w.pair_proj = P(p + "pair_proj");
        w.gate = P(p + "gate");
        w.gate_T = P(p + "gate_T");
        w.gate_b = P(p + "gate_b");
        w.vmix = c.vector_channels ? P(p + "vmix") : nullptr;
        w.up1_f = P(p + "up1_f");
        w.up1_fT = P(p + "up1_fT");
        w.up1_b = P(p + "up1_b");
        w.up2 = P(p + "up2");
        w.up2_T = P(p + "up2_T");
        w.up2_b = P(p + "up2_b");
    }
}

int MessagePlan::add(Arena &ar, size_t bytes) {
    offs.push_back(ar.add(bytes));
    return int(offs.size()) - 1;
}

MessagePlan plan_messages(ModelImpl &m, Arena &ar, int N, int64_t E) {
    MessagePlan p;
    const rune_model_config &c = m.cfg;
    if (c.family != RUNE_FAMILY_MOBIUS || c.message_layers == 0) return p;
    if (c.message_mode == RUNE_MESSAGE_EQUIVARIANT) return plan_equivariant(m, ar, N, E);
    const size_t n = size_t(N), e = size_t(std::max<int64_t>(E, 1));
    const int H = c.hidden_dim, D = c.message_dim, vc = c.vector_channels;
    const int NP = H + vc, NG = c.message_groups + vc, L = c.message_layers;
    p.N = N;
    p.E = E;
    p.ldrb = (c.message_basis_size + 3) & ~3;
    p.o_gd = ar.add(16 * e);
    p.o_dmom = 0;
    p.i_rb = p.add(ar, 4 * e * p.ldrb);
    p.i_fc = p.add(ar, 4 * e);
    p.i_pair = p.add(ar, 4 * e);
    p.i_dv = p.add(ar, 16 * e);
    // the fused edge MLP keeps pre-activations and their adjoints in registers
    const bool fusable = mp_edge_fusable(D, NG, c.message_basis_size);
    const size_t ed = fusable ? 1 : e;
    // the fused edge reverses run on the side stream: each block keeps its gate
    // adjoints, and their dE/dd goes to its own accumulator
    const bool side = fusable && m.side;
    if (side) p.i_dd = p.add(ar, 4 * e);
    for (int b = 0; b < L; ++b) {
        BlockBuffers bb;
        bb.h_out = p.add(ar, 4 * n * H);
        bb.rin = p.add(ar, 4 * n);
        bb.vs = p.add(ar, 4 * n * NP);
        bb.ue = p.add(ar, 4 * ed * D);
        bb.gv = p.add(ar, 4 * e * NG);
        if (side) bb.dgv = p.add(ar, 4 * e * NG);
        bb.msg = p.add(ar, 4 * n * H);
        bb.rm = p.add(ar, 4 * n);
        bb.vsum = p.add(ar, 4 * n * 3 * std::max(vc, 1));
        bb.mixed = p.add(ar, 4 * n * 3 * std::max(vc, 1));
        bb.uin = p.add(ar, 4 * n * NP);
        bb.u1 = p.add(ar, 4 * n * D);
        bb.z1 = p.add(ar, 4 * n * D);
        p.blocks.push_back(bb);
    }
    p.t_dz1 = p.add(ar, 4 * n * D);
    p.t_duin = p.add(ar, 4 * n * NP);
    p.t_dmsg = p.add(ar, 4 * n * H);
    p.t_dvsum = p.add(ar, 4 * n * 3 * std::max(vc, 1));
    p.t_dgv = p.add(ar, 4 * e * NG);
    p.t_due = p.add(ar, 4 * ed * D);
    p.t_drb = p.add(ar, 4 * ed * p.ldrb);
    p.t_dvs = p.add(ar, 4 * n * NP);
    p.t_dz = p.add(ar, 4 * n * H);
    p.t_dh0 = p.add(ar, 4 * n * H);
    p.t_dh1 = p.add(ar, 4 * n * H);
    return p;
}

static int edge_grid(int64_t E) { return ceil_div(std::max<int64_t>(E, 1), 256); }

void edge_prep(ModelImpl &m, MessagePlan &p, const Records &r, const int32_t *types,
               hipStream_t s, float *harm, const float *scale, int lq, int nq) {
    if (p.E == 0) return;
    EdgePrepArgs a{};
    a.r = r;
    a.E = p.E;
    a.types = types;
    a.n_types = m.cfg.n_types;
    a.cutoff = float(m.cfg.message_cutoff);
    a.kb = m.cfg.message_basis_size;
    a.ldrb = p.ldrb;
    a.rb = p.at(p.i_rb);
    a.rbd = p.i_rbd >= 0 ? p.at(p.i_rbd) : nullptr;
    a.fc = p.at(p.i_fc);
    a.pair = reinterpret_cast<int32_t *>(p.at(p.i_pair));
    a.dv = reinterpret_cast<float4 *>(p.at(p.i_dv));
    a.dd = p.i_dd >= 0 ? p.at(p.i_dd) : nullptr;
    a.harm = harm;
    a.scale = scale;
    a.lq = lq;
    a.nq = nq;
    a.z = m.desc.z;
    for (int k = 0; k < kMaxL + 2; ++k) a.z_off[k] = m.desc.z_off[k];
    const size_t lds = sizeof(float) * 256 * ((a.rbd ? 2 : 1) * size_t(a.ldrb) + (harm ? nq : 0));
    static bool raised = false;   // LDS beyond the default dynamic limit (large nq)
    if (!raised) {
        RUNE_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_edge_prep),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           160 * 1024));
        raised = true;
    }
    hipLaunchKernelGGL(k_edge_prep, dim3(edge_grid(p.E)), dim3(256), lds, s, a);
    RUNE_HIP_CHECK(hipGetLastError());
}

void edge_rb_backward(ModelImpl &m, MessagePlan &p, const Records &r, const float *drb, int ld,
                      hipStream_t s) {
    if (p.E == 0) return;
    hipLaunchKernelGGL(k_edge_rb_backward, dim3(edge_grid(p.E)), dim3(256), 0, s, p.E, r,
                       p.at(p.i_fc), drb, ld, m.cfg.message_basis_size,
                       float(m.cfg.message_cutoff), reinterpret_cast<float4 *>(p.at(p.i_dv)));
    RUNE_HIP_CHECK(hipGetLastError());
}

void edge_direct(MessagePlan &p, const Records &r, hipStream_t s) {
    if (p.E == 0) return;
    hipLaunchKernelGGL(k_edge_direct, dim3(edge_grid(p.E)), dim3(256), 0, s, p.E, r,
                       reinterpret_cast<const float4 *>(p.at(p.i_dv)),
                       p.i_dd >= 0 ? p.at(p.i_dd) : nullptr, p.g_direct);
    RUNE_HIP_CHECK(hipGetLastError());
}

static MpArgs mp_args(ModelImpl &m, MessagePlan &p, const Records &r, int b) {
    const rune_model_config &c = m.cfg;
    const BlockBuffers &bb = p.blocks[b];
    MpArgs a{};
    a.r = r;
    a.H = c.hidden_dim;
    a.G = c.message_groups;
    a.vc = c.vector_channels;
    a.NG = a.G + a.vc;
    a.NP = a.H + a.vc;
    a.eps = float(c.norm_eps);
    a.fc = p.at(p.i_fc);
    a.gv = p.at(bb.gv);
    a.vs = p.at(bb.vs);
    a.vmix = m.msg[b].vmix;
    a.msg = p.at(bb.msg);
    a.rm = p.at(bb.rm);
    a.vsum = p.at(bb.vsum);
    a.mixed = p.at(bb.mixed);
    a.uin = p.at(bb.uin);
    a.duin = p.at(p.t_duin);
    a.dmsg = p.at(p.t_dmsg);
    a.dvsum = p.at(p.t_dvsum);
    a.dgv = bb.dgv >= 0 ? p.at(bb.dgv) : p.at(p.t_dgv);
    a.dv = reinterpret_cast<float4 *>(p.at(p.i_dv));
    a.dvs = p.at(p.t_dvs);
    a.cutoff = float(c.message_cutoff);
    return a;
}

static MpEdgeArgs mp_edge_args(ModelImpl &m, MessagePlan &p, const MessageWeights &w,
                               int64_t E) {
    const rune_model_config &c = m.cfg;
    MpEdgeArgs a{};
    a.E = E;
    a.rb = p.at(p.i_rb);
    a.ldrb = p.ldrb;
    a.kb = c.message_basis_size;
    a.KP = w.ld_edge_x;
    a.pair = reinterpret_cast<const int32_t *>(p.at(p.i_pair));
    a.Wx = w.edge_x;
    a.P = w.pair_proj;
    a.Wg = w.gate;
    a.gb = w.gate_b;
    a.D = c.message_dim;
    a.NG = w.NG;
    a.act = c.activation;
    return a;
}

// The record-only forward work of the MP blocks: the edge features (basis,
// cutoff, pair index; message.py:108-110) and every block's edge MLP (gate
// logits from the features and the pair row, message.py:160, :178), none of
// which reads a node state.
static void mp_record_forward(ModelImpl &m, MessagePlan &p, const Records &r,
                              const int32_t *types, hipStream_t s) {
    const rune_model_config &c = m.cfg;
    const int D = c.message_dim, act = c.activation;
    const int64_t E = p.E;
    {
        Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
        edge_prep(m, p, r, types, s, nullptr, nullptr, 0, 0);
    }
    for (int b = 0; b < c.message_layers && E > 0; ++b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        bool fused = false;
        {
            Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
            MpEdgeArgs ea = mp_edge_args(m, p, w, E);
            ea.gv = p.at(bb.gv);
            fused = mp_edge_fused(ea, false, s);
        }
        if (!fused) {
            Epilogue e1;
            e1.gtab[0] = w.pair_proj;
            e1.gidx[0] = reinterpret_cast<const int32_t *>(p.at(p.i_pair));
            e1.gld[0] = D;
            {
                Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                gemm(int(E), D, w.KX, p.at(p.i_rb), p.ldrb, w.edge_x, w.ld_edge_x, p.at(bb.ue),
                     D, e1, s);
            }
            // the gate GEMM activates the pre-activations as it stages them
            Epilogue e2;
            e2.bias = w.gate_b;
            e2.a_act = act;
            {
                Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                gemm(int(E), w.NG, D, p.at(bb.ue), D, w.gate, D, p.at(bb.gv), w.NG, e2, s);
            }
        }
    }
    RUNE_HIP_CHECK(hipGetLastError());
}

bool messages_records_ahead(ModelImpl &m, MessagePlan &p, const Records &r,
                            const int32_t *types, hipStream_t s) {
    const rune_model_config &c = m.cfg;
    if (c.family != RUNE_FAMILY_MOBIUS || c.message_layers == 0 ||
        c.message_mode == RUNE_MESSAGE_EQUIVARIANT || !m.side)
        return false;
    RUNE_HIP_CHECK(hipEventRecord(m.fork_ev, s));
    RUNE_HIP_CHECK(hipStreamWaitEvent(m.side, m.fork_ev, 0));
    p.records_ready = true;   // set first: a failed launch below still joins
    mp_record_forward(m, p, r, types, m.side);
    return true;
}

float *messages_forward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                        const int32_t *types, const float *moments, float *h, hipStream_t s,
                        bool keep) {
    const rune_model_config &c = m.cfg;
    if (c.family != RUNE_FAMILY_MOBIUS || c.message_layers == 0) return h;
    if (c.message_mode == RUNE_MESSAGE_EQUIVARIANT)
        return equivariant_forward(m, p, lp, r, types, moments, h, s, keep);
    const int N = p.N, H = c.hidden_dim, D = c.message_dim, act = c.activation;
    (void)keep;
    if (!p.records_ready) mp_record_forward(m, p, r, types, s);
    float *cur = h;
    for (int b = 0; b < c.message_layers; ++b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        Epilogue e0;
        e0.rms_out = p.at(bb.rin);   // input RMSNorm, formed by the GEMM
        e0.rms_eps = float(c.norm_eps);
        gemm(N, w.NP, H, cur, H, w.node_f, H, p.at(bb.vs), w.NP, e0, s);
        MpArgs a = mp_args(m, p, r, b);
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            const dim3 grid(ceil_div(N, 4)), block(256);
            switch (mp_columns(H, c.message_groups, w.NP)) {
            case 4: hipLaunchKernelGGL(k_mp_aggregate_c<4>, grid, block, 0, s, a); break;
            case 8: hipLaunchKernelGGL(k_mp_aggregate_c<8>, grid, block, 0, s, a); break;
            case 16: hipLaunchKernelGGL(k_mp_aggregate_c<16>, grid, block, 0, s, a); break;
            default: hipLaunchKernelGGL(k_mp_aggregate, grid, block, 0, s, a);
            }
        }
        RUNE_HIP_CHECK(hipGetLastError());
        Epilogue e3;
        e3.bias = w.up1_b;
        e3.pre = p.at(bb.u1);
        e3.ldp = D;
        e3.act = act;
        gemm(N, D, w.NP, p.at(bb.uin), w.NP, w.up1_f, w.NP, p.at(bb.z1), D, e3, s);
        Epilogue e4;
        e4.bias = w.up2_b;
        e4.residual = cur;
        e4.ldr = H;
        gemm(N, H, D, p.at(bb.z1), D, w.up2, D, p.at(bb.h_out), H, e4, s);
        p.block_input.push_back(cur);
        cur = p.at(bb.h_out);
    }
    return cur;
}

float *messages_backward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                         const int32_t *types, const float *moments, float *dh, hipStream_t s) {
    const rune_model_config &c = m.cfg;
    if (c.family != RUNE_FAMILY_MOBIUS || c.message_layers == 0) return dh;
    if (c.message_mode == RUNE_MESSAGE_EQUIVARIANT)
        return equivariant_backward(m, p, lp, r, types, moments, dh, s);
    const int N = p.N, H = c.hidden_dim, D = c.message_dim, act = c.activation;
    const int64_t E = p.E;
    float *cur = dh;
    bool tail_side = false;   // edge reverses enqueued on the side stream
    for (int b = c.message_layers - 1; b >= 0; --b) {
        const MessageWeights &w = m.msg[b];
        const BlockBuffers &bb = p.blocks[b];
        const float *hin = p.block_input[b];
        Epilogue e0;
        e0.dact_from = p.at(bb.u1);
        e0.ldu = D;
        e0.dact = act;
        gemm(N, D, H, cur, H, w.up2_T, H, p.at(p.t_dz1), D, e0, s);
        Epilogue e1;
        gemm(N, w.NP, D, p.at(p.t_dz1), D, w.up1_fT, D, p.at(p.t_duin), w.NP, e1, s);
        MpArgs a = mp_args(m, p, r, b);
        hipLaunchKernelGGL(k_mp_node_backward, dim3(N), dim3(kWave), 0, s, a);
        const size_t lds = sizeof(float) * 4 * kMpSlots * (H + 1);
        const dim3 grid(ceil_div(N, 4)), block(256);
        const int ch = mp_columns(H, c.message_groups, w.NP);
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            switch (ch) {
            case 4: hipLaunchKernelGGL(k_mp_edge_backward_c<4>, grid, block, 0, s, a); break;
            case 8: hipLaunchKernelGGL(k_mp_edge_backward_c<8>, grid, block, 0, s, a); break;
            case 16: hipLaunchKernelGGL(k_mp_edge_backward_c<16>, grid, block, 0, s, a); break;
            default: hipLaunchKernelGGL(k_mp_edge_backward, grid, block, lds, s, a);
            }
        }
        {
            Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
            switch (ch) {
            case 4: hipLaunchKernelGGL(k_mp_neighbor_backward_c<4>, grid, block, 0, s, a); break;
            case 8: hipLaunchKernelGGL(k_mp_neighbor_backward_c<8>, grid, block, 0, s, a); break;
            case 16:
                hipLaunchKernelGGL(k_mp_neighbor_backward_c<16>, grid, block, 0, s, a);
                break;
            default: hipLaunchKernelGGL(k_mp_neighbor_backward, grid, block, 0, s, a);
            }
        }
        RUNE_HIP_CHECK(hipGetLastError());
        if (E > 0) {
            // the edge reverse feeds only the geometric derivative, so with a
            // block-owned dgv it runs on the side stream beside the node chain
            hipStream_t es = s;
            if (bb.dgv >= 0) {
                RUNE_HIP_CHECK(hipEventRecord(m.fork_ev, s));
                RUNE_HIP_CHECK(hipStreamWaitEvent(m.side, m.fork_ev, 0));
                es = m.side;
                tail_side = true;
            }
            bool fused = false;
            {
                Span sp(m, RUNE_GROUP_EDGE_GEMM, es);
                MpEdgeArgs ea = mp_edge_args(m, p, w, E);
                ea.dgv = a.dgv;
                ea.fc = p.at(p.i_fc);
                ea.vec = r.vec;
                ea.dv = reinterpret_cast<float4 *>(p.at(p.i_dv));
                ea.dd = bb.dgv >= 0 ? p.at(p.i_dd) : nullptr;
                ea.cutoff = float(c.message_cutoff);
                fused = mp_edge_fused(ea, true, es);
            }
            RUNE_REQUIRE(fused || es == s, RUNE_ERR_STATE, "internal: unfused side reverse");
            if (!fused) {
                Epilogue e2;
                e2.dact_from = p.at(bb.ue);
                e2.ldu = D;
                e2.dact = act;
                {
                    Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                    gemm(int(E), D, w.NG, p.at(p.t_dgv), w.NG, w.gate_T, w.NG, p.at(p.t_due), D,
                         e2, s);
                }
                Epilogue e3;
                {
                    Span sp(m, RUNE_GROUP_EDGE_GEMM, s);
                    gemm(int(E), w.KX, D, p.at(p.t_due), D, w.edge_xT, D, p.at(p.t_drb), p.ldrb,
                         e3, s);
                }
            }
            if (!fused) {   // the fused reverse adds this contraction itself
                Span sp(m, RUNE_GROUP_EDGE_KERNELS, s);
                edge_rb_backward(m, p, r, p.at(p.t_drb), p.ldrb, s);
            }
        }
        Epilogue e4;
        gemm(N, H, w.NP, p.at(p.t_dvs), w.NP, w.node_fT, w.NP, p.at(p.t_dz), H, e4, s);
        float *next = (cur == p.at(p.t_dh0)) ? p.at(p.t_dh1) : p.at(p.t_dh0);
        rms_backward(N, H, hin, H, p.at(bb.rin), p.at(p.t_dz), H, cur, H, next, H, s);
        cur = next;
    }
    // the direct edge gradient after the last reverse (and after every
    // contribution of the node chain to dv)
    hipStream_t ts = s;
    if (tail_side) {
        RUNE_HIP_CHECK(hipEventRecord(m.fork_ev, s));
        RUNE_HIP_CHECK(hipStreamWaitEvent(m.side, m.fork_ev, 0));
        ts = m.side;
    }
    {
        Span sp(m, RUNE_GROUP_EDGE_KERNELS, ts);
        edge_direct(p, r, ts);
    }
    p.g_direct_used = E > 0;
    return cur;
}

}  // namespace rune
