// K2 / K3: descriptor forward and its geometry reverse pass (+ ZBL).
//
// One 64-lane wavefront per centre atom.  The forward kernel evaluates the
// Chebyshev radial basis and the real angular polynomials per edge and
// reduces them into q (rune/mobius/descriptor.py:822-911) in a fixed order;
// the reverse kernel forms dE/ds from dE/dq (force.py:28-133), contracts it
// with the per-edge basis Jacobians (force.py:165-243) and adds the ZBL pair
// term (zbl.py:92-141).  No atomics: every output has one writer.
#include <cmath>

#include "cubic.hpp"
#include "kernels.hpp"

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

// f_k(r) of descriptor.py:377-414, k < k_max.
template <int KMAX>
__device__ inline void chebyshev(float r, float rc, int k_max, float *f) {
    float rcinv = 1.0f / rc;
    float arg = kPi * r * rcinv;
    float fc = 0.5f * cosf(arg) + 0.5f;
    float rs = r * rcinv - 1.0f;
    float x = 2.0f * rs * rs - 1.0f;
    f[0] = fc;
    float t2 = 1.0f, t1 = x;
#pragma unroll
    for (int k = 1; k < KMAX; ++k) {
        if (k >= k_max) break;
        float t = (k == 1) ? x : 2.0f * x * t1 - t2;
        if (k > 1) {
            t2 = t1;
            t1 = t;
        }
        f[k] = 0.5f * (t + 1.0f) * fc;
    }
}

// f_k(r) and d f_k / d r.
template <int KMAX>
__device__ inline void chebyshev_d(float r, float rc, int k_max, float *f, float *fp) {
    float rcinv = 1.0f / rc;
    float arg = kPi * r * rcinv;
    float fc = 0.5f * cosf(arg) + 0.5f;
    float fcp = -0.5f * kPi * rcinv * sinf(arg);
    float rs = r * rcinv - 1.0f;
    float x = 2.0f * rs * rs - 1.0f;
    float dxdr = 4.0f * rs * rcinv;
    f[0] = fc;
    fp[0] = fcp;
    float t2 = 1.0f, t1 = x;      // T_{k-2}, T_{k-1}
    float u2 = 1.0f, u1 = 2.0f * x;  // U_{k-2}, U_{k-1}
#pragma unroll
    for (int k = 1; k < KMAX; ++k) {
        if (k >= k_max) break;
        if (k == 1) {
            float core = 0.5f * (x + 1.0f);
            f[1] = core * fc;
            fp[1] = 0.5f * dxdr * fc + core * fcp;
        } else {
            float tn = 2.0f * x * t1 - t2;
            float un = 2.0f * x * u1 - u2;
            float core = 0.5f * (tn + 1.0f);
            f[k] = core * fc;
            fp[k] = 0.5f * float(k) * u1 * dxdr * fc + core * fcp;
            t2 = t1;
            t1 = tn;
            u2 = u1;
            u1 = un;
        }
    }
}

// Powers of the unit vector are formed as running products while the (L, |m|)
// loops advance, never stored in an array: a per-lane array indexed by a
// runtime order would live in scratch memory.
//   (x + iy)^m:  w_m = w_{m-1} * (x + iy), w_0 = 1
//   z^q:         z^q = z^{q-1} * z, z^0 = 1
__device__ inline void next_w(float x, float y, float &wr, float &wi) {
    float r = wr * x - wi * y;
    wi = wr * y + wi * x;
    wr = r;
}

// sum_k c[k] f[k] over one padded c-table row (16-byte loads; the padding is
// zero and f is zero there, so the sum equals the unpadded one term by term).
template <int KMAX>
__device__ inline float row_dot(const float *row, int k4, const float *f) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < KMAX / 4; ++q) {
        if (4 * q >= k4) break;
        const float4 c = r4[q];
        a += c.x * f[4 * q];
        a += c.y * f[4 * q + 1];
        a += c.z * f[4 * q + 2];
        a += c.w * f[4 * q + 3];
    }
    return a;
}

// z-polynomial of order L, |m| = n1 (descriptor.py:601-613) and d/dz.
__device__ inline void zpoly(const DescTables &t, int L, int n1, float z, float &zf,
                             float &zfp) {
    const float *Z = t.z + t.z_off[L] + n1 * (L + 1);
    int q = (L + n1) & 1;
    float zq = q ? z : 1.0f;   // z^q
    float zq1 = 1.0f;          // z^(q-1), used once q > 0
    zf = 0.0f;
    zfp = 0.0f;
    for (; q <= L - n1; q += 2) {
        zf += Z[q] * zq;
        if (q > 0) zfp += float(q) * Z[q] * zq1;
        zq1 = zq * z;
        zq = zq1 * z;
    }
}

// One channel's moments s[0..kCubicComps) in registers (zero past nlm).
__device__ inline void cubic_moments(const float *s, int nlm, float (&sr)[kCubicComps]) {
#pragma unroll
    for (int c = 0; c < kCubicComps; ++c) sr[c] = c < nlm ? s[c] : 0.0f;
}

// Invariant idx of the q layout (L = 1..l_max, then q222, q1111, q112, q123,
// q233, q134 as enabled; descriptor.py:650-725) of one channel's moments s.
__device__ float invariant_one(const DescTables &t, const float *s, int idx) {
    if (idx < t.l_max) {
        const int L = idx + 1, st = L * L - 1;
        const float q = t.c3b[st] * s[st] * s[st];
        float acc = 0.0f;
        for (int c = 1; c <= 2 * L; ++c) acc += t.c3b[st + c] * s[st + c] * s[st + c];
        return q + 2.0f * acc;
    }
    int kind = 0;
    for (int k = idx - t.l_max; kind < 6; ++kind)
        if (t.has_q[kind] && k-- == 0) break;
    if (kind == 0) {
        const float *c = t.c4b;
        const float s3 = s[3], s4 = s[4], s5 = s[5], s6 = s[6], s7 = s[7];
        return c[0] * s3 * s3 * s3 + c[1] * s3 * (s4 * s4 + s5 * s5) +
               c[2] * s3 * (s6 * s6 + s7 * s7) + c[3] * s6 * (s5 * s5 - s4 * s4) +
               c[4] * s4 * s5 * s7;
    }
    if (kind == 1) {
        const float *c = t.c5b;
        const float a = s[0] * s[0], b = s[1] * s[1] + s[2] * s[2];
        return c[0] * a * a + c[1] * a * b + c[2] * b * b;
    }
    if (kind == 2) {
        const float *c = t.c4b2;
        const float a = s[0], b = s[1], cc = s[2], d = s[3], e = s[4], f = s[5], g = s[6],
                    h = s[7];
        return c[0] * a * a * d + c[1] * a * (b * e + cc * f) + c[2] * d * (b * b + cc * cc) +
               c[3] * g * (b * b - cc * cc) + c[4] * b * cc * h;
    }
    float sr[kCubicComps];
    cubic_moments(s, t.nlm, sr);
    return kind == 3 ? cubic_value<0>(sr) : kind == 4 ? cubic_value<1>(sr) : cubic_value<2>(sr);
}

// q of every angular channel (moments sL[n * nlm + c]): one output per lane,
// out[idx * na + n] for invariant idx of channel n.
__device__ void invariants_all(const DescTables &t, const float *sL, float *out, int lane) {
    const int na = t.na, nlm = t.nlm;
    for (int o = lane; o < na * t.num_L; o += kWave) {
        const int idx = o / na, n = o - idx * na;
        out[o] = invariant_one(t, sL + n * nlm, idx);
    }
}

// dE/ds_c of one channel from its order and four/five-body invariants: sum
// over them of dq[idx * stride] * d q_idx / d s_c (force.py:28-133).
__device__ float invariant_grad_one(const DescTables &t, const float *s, const float *dq,
                                    int stride, int c) {
    float w = 0.0f;
    int L = 1;
    while ((L + 1) * (L + 1) - 1 <= c) ++L;   // c in [L^2 - 1, (L + 1)^2 - 1)
    const int st = L * L - 1;
    if (L <= t.l_max) w += dq[stride * (L - 1)] * ((c == st ? 2.0f : 4.0f) * t.c3b[c] * s[c]);
    int idx = t.l_max;
    if (t.has_q[0]) {
        const float *k = t.c4b;
        const float g = dq[stride * idx++];
        const float s20 = s[3], s21r = s[4], s21i = s[5], s22r = s[6], s22i = s[7];
        if (c == 3)
            w += g * (3.0f * k[0] * s20 * s20 + k[1] * (s21r * s21r + s21i * s21i) +
                      k[2] * (s22r * s22r + s22i * s22i));
        else if (c == 4)
            w += g * (2.0f * k[1] * s20 * s21r - 2.0f * k[3] * s22r * s21r + k[4] * s21i * s22i);
        else if (c == 5)
            w += g * (2.0f * k[1] * s20 * s21i + 2.0f * k[3] * s22r * s21i + k[4] * s21r * s22i);
        else if (c == 6)
            w += g * (2.0f * k[2] * s20 * s22r + k[3] * (s21i * s21i - s21r * s21r));
        else if (c == 7)
            w += g * (2.0f * k[2] * s20 * s22i + k[4] * s21r * s21i);
    }
    if (t.has_q[1]) {
        const float *k = t.c5b;
        const float g = dq[stride * idx++];
        if (c <= 2) {
            const float s0 = s[0], s1 = s[1], s2 = s[2];
            const float a = s0 * s0, b = s1 * s1 + s2 * s2;
            const float factor = k[1] * a + 2.0f * k[2] * b;
            if (c == 0)
                w += g * (2.0f * s0 * (2.0f * k[0] * a + k[1] * b));
            else
                w += g * 2.0f * s[c] * factor;
        }
    }
    if (t.has_q[2]) {
        const float *k = t.c4b2;
        const float g = dq[stride * idx++];
        const float a = s[0], b = s[1], cc = s[2], d = s[3], e = s[4], f = s[5], gg = s[6],
                    h = s[7];
        if (c == 0)
            w += g * (2.0f * k[0] * a * d + k[1] * (b * e + cc * f));
        else if (c == 1)
            w += g * (k[1] * a * e + 2.0f * k[2] * d * b + 2.0f * k[3] * gg * b + k[4] * cc * h);
        else if (c == 2)
            w += g * (k[1] * a * f + 2.0f * k[2] * d * cc - 2.0f * k[3] * gg * cc + k[4] * b * h);
        else if (c == 3)
            w += g * (k[0] * a * a + k[2] * (b * b + cc * cc));
        else if (c == 4)
            w += g * k[1] * a * b;
        else if (c == 5)
            w += g * k[1] * a * cc;
        else if (c == 6)
            w += g * k[3] * (b * b - cc * cc);
        else if (c == 7)
            w += g * k[4] * b * cc;
    }
    return w;
}

// WL[n * nlm + c] += dE/ds_c of channel n for every (n, c): one output per
// lane for the order and four/five-body invariants, then one channel per
// lane for the cubic invariants (their unrolled term lists read the moments
// from registers and update the row at constant offsets).
template <bool kRegCubic = false, int STEP = kWave>
__device__ void invariant_gradient_all(const DescTables &t, const float *sL, const float *dq,
                                       float *WL, int lane) {
    const int na = t.na, nlm = t.nlm;
    for (int o = lane; o < na * nlm; o += STEP) {
        const int n = o / nlm, c = o - n * nlm;
        WL[o] += invariant_grad_one(t, sL + n * nlm, dq + n, na, c);
    }
    if (!(t.has_q[3] || t.has_q[4] || t.has_q[5])) return;
    __syncthreads();
    for (int n = lane; n < na; n += STEP) {
        float sr[kCubicComps];
        cubic_moments(sL + n * nlm, nlm, sr);
        // kRegCubic: accumulate in registers (no LDS read-modify-write chain,
        // more registers: the variant for grids too small to fill the chip)
        float wr[kCubicComps];
#pragma unroll
        for (int c = 0; c < kCubicComps; ++c) wr[c] = 0.0f;
        float *w = kRegCubic ? wr : WL + n * nlm;
        int idx = t.l_max + t.has_q[0] + t.has_q[1] + t.has_q[2];
        if (t.has_q[3]) cubic_grad<0>(sr, dq[n + na * idx++], w, nlm);
        if (t.has_q[4]) cubic_grad<1>(sr, dq[n + na * idx++], w, nlm);
        if (t.has_q[5]) cubic_grad<2>(sr, dq[n + na * idx++], w, nlm);
        if constexpr (kRegCubic) {
#pragma unroll
            for (int c = 0; c < kCubicComps; ++c)
                if (c < nlm) WL[n * nlm + c] += wr[c];
        }
    }
}

// KR / KA: basis values of a lane's record, NR: radial channels, NO: moment
// outputs per lane (register arrays sized for the model, so the compact
// instantiation keeps occupancy up).
// kMfma: the moment sums of a round on the matrix cores (na <= 16 channels,
// nlm <= 32 components): M[n][c] += sum_k gn[k][n] b[k][c] as
// v_mfma_f32_16x16x4f32 over four records at a time, two 16-column tiles.
template <int KR, int KA, int NR, int NO, int CH = kWave, bool kMfma = false>
__global__ void __launch_bounds__(kWave) k_descriptor_forward(DescTables t, Records r,
                                                              const int32_t *types, float *q,
                                                              int ldq, float *moments) {
    extern __shared__ float lds[];
    const int nlm = t.nlm, na = t.na, nout = na * nlm;
    float *gnL = lds;                          // [CH][na+1]
    float *bL = gnL + CH * (na + 1);           // [CH][nlm+1]
    float *sL = lds;                           // [na*nlm], after the record rounds
    const int i = blockIdx.x;
    const int lane = threadIdx.x;
    const int ti = types[i];
    const int rb = r.view[4 * i], re = r.view[4 * i + 1];
    const int ab = r.view[4 * i + 2], ae = r.view[4 * i + 3];

    // radial channels
    float qr[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) qr[n] = 0.0f;
    for (int e = rb + lane; e < re; e += kWave) {
        float4 v = r.vec[e];
        int tj = types[r.nbr[e]];
        float f[KR] = {};
        chebyshev<KR>(v.w, t.rc_r, t.kr, f);
        const float *row = t.c_radial + size_t(ti * t.n_types + tj) * t.nr * t.kr4;
#pragma unroll
        for (int n = 0; n < NR; ++n) {
            if (n >= t.nr) break;
            qr[n] += row_dot<KR>(row + n * t.kr4, t.kr4, f);
        }
    }
#pragma unroll
    for (int n = 0; n < NR; ++n) {
        if (n >= t.nr) break;
        float v = wave_sum(qr[n]);
        if (lane == 0) q[size_t(i) * ldq + n] = v;
    }

    // angular moments s[n][lm] = sum_e gn[e][n] b[e][lm], CH records (lanes)
    // per round
    float acc[NO];
#pragma unroll
    for (int j = 0; j < NO; ++j) acc[j] = 0.0f;
    floatx4_t mt[2] = {floatx4_t{0.0f, 0.0f, 0.0f, 0.0f}, floatx4_t{0.0f, 0.0f, 0.0f, 0.0f}};
    const int mr = lane & 15, mg = lane >> 4;   // MFMA operand row / k group
    for (int base = ab; base < ae; base += CH) {
        int e = base + lane;
        float *gl = gnL + lane * (na + 1);
        float *bl = bL + lane * (nlm + 1);
        if (lane < CH && e < ae) {
            float4 v = r.vec[e];
            int tj = types[r.nbr[e]];
            float f[KA] = {};
            chebyshev<KA>(v.w, t.rc_a, t.ka, f);
            const float *row = t.c_angular + size_t(ti * t.n_types + tj) * t.na * t.ka4;
            for (int n = 0; n < na; ++n) gl[n] = row_dot<KA>(row + n * t.ka4, t.ka4, f);
            float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
            const float ux = v.x * inv, uy = v.y * inv, uz = v.z * inv;
            int idx = 0;
            for (int L = 1; L <= t.l_max; ++L) {
                float wr = 1.0f, wi = 0.0f;   // (x + iy)^n1
                for (int n1 = 0; n1 <= L; ++n1) {
                    float zf, zfp;
                    zpoly(t, L, n1, uz, zf, zfp);
                    if (n1 == 0) {
                        bl[idx++] = zf;
                    } else {
                        next_w(ux, uy, wr, wi);
                        bl[idx++] = zf * wr;
                        bl[idx++] = zf * wi;
                    }
                }
            }
        } else if (lane < CH) {
            for (int n = 0; n < na; ++n) gl[n] = 0.0f;
            for (int c = 0; c < nlm; ++c) bl[c] = 0.0f;
        }
        __syncthreads();
        int cnt = min(CH, ae - base);
        if constexpr (kMfma) {
            // lane l feeds A[n = l%16][k] = gn[k][n] and B[k][c = 16 t + l%16] =
            // b[k][c] for record k = k0 + l/16; zero past na, nlm and cnt
            for (int k0 = 0; k0 < cnt; k0 += 4) {
                const int k = k0 + mg;
                const bool kin = k < cnt;
                const float av = kin && mr < na ? gnL[k * (na + 1) + mr] : 0.0f;
                const float b0 = kin && mr < nlm ? bL[k * (nlm + 1) + mr] : 0.0f;
                const float b1 = kin && 16 + mr < nlm ? bL[k * (nlm + 1) + 16 + mr] : 0.0f;
                mt[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b0, mt[0], 0, 0, 0);
                mt[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b1, mt[1], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NO; ++j) {
                int o = lane + kWave * j;
                if (o >= nout) break;
                int n = o / nlm, c = o - n * nlm;
                float a = 0.0f;
                for (int k = 0; k < cnt; ++k) a += gnL[k * (na + 1) + n] * bL[k * (nlm + 1) + c];
                acc[j] += a;
            }
        }
        __syncthreads();
    }
    if constexpr (kMfma) {
        // accumulator v of lane l is M[n = 4 (l/16) + v][c = 16 t + l%16]
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = 4 * mg + v, c = 16 * tt + mr;
                if (n < na && c < nlm) {
                    sL[n * nlm + c] = mt[tt][v];
                    moments[size_t(i) * nout + n * nlm + c] = mt[tt][v];
                }
            }
        __syncthreads();
        invariants_all(t, sL, q + size_t(i) * ldq + t.nr, lane);
        return;
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
        int o = lane + kWave * j;
        if (o >= nout) break;
        sL[o] = acc[j];
        moments[size_t(i) * nout + o] = acc[j];
    }
    __syncthreads();
    invariants_all(t, sL, q + size_t(i) * ldq + t.nr, lane);
}

// Two centres per wave (lanes 0-31 centre 2b, lanes 32-63 centre 2b + 1) for
// sparse lists (at most about 32 records per centre, e.g. NEP on a
// 13,824-atom cell): the arithmetic of k_descriptor_forward over half-waves,
// with record rounds of 32 per half, so a launch has half the waves and a
// wave's lanes are not mostly idle.  Sums over a half-wave stay in it
// (shuffle offsets below 32).
template <int KR, int KA, int NR, int NO2>
__global__ void __launch_bounds__(kWave) k_descriptor_forward_pair(DescTables t, Records r,
                                                                   const int32_t *types, float *q,
                                                                   int ldq, float *moments) {
    extern __shared__ float lds[];
    constexpr int H = kWave / 2;
    const int nlm = t.nlm, na = t.na, nout = na * nlm;
    const int lane = threadIdx.x, half = lane >> 5, hl = lane & (H - 1);
    const int i = 2 * int(blockIdx.x) + half;
    const bool valid = i < r.n_atoms;
    const int ic = valid ? i : r.n_atoms - 1;
    const int hstride = max(H * (na + nlm + 2), nout);
    float *gnL = lds + half * hstride;   // [H][na+1]
    float *bL = gnL + H * (na + 1);      // [H][nlm+1]
    float *sL = gnL;                     // [na*nlm], after the record rounds
    const int ti = types[ic];
    const int rb = r.view[4 * ic], re = valid ? r.view[4 * ic + 1] : rb;
    const int ab = r.view[4 * ic + 2], ae = valid ? r.view[4 * ic + 3] : ab;

    // radial channels
    float qr[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) qr[n] = 0.0f;
    for (int e = rb + hl; e < re; e += H) {
        float4 v = r.vec[e];
        int tj = types[r.nbr[e]];
        float f[KR] = {};
        chebyshev<KR>(v.w, t.rc_r, t.kr, f);
        const float *row = t.c_radial + size_t(ti * t.n_types + tj) * t.nr * t.kr4;
#pragma unroll
        for (int n = 0; n < NR; ++n) {
            if (n >= t.nr) break;
            qr[n] += row_dot<KR>(row + n * t.kr4, t.kr4, f);
        }
    }
#pragma unroll
    for (int n = 0; n < NR; ++n) {
        if (n >= t.nr) break;
        float v = qr[n];
#pragma unroll
        for (int off = H / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
        if (hl == 0 && valid) q[size_t(i) * ldq + n] = v;
    }

    // angular moments, rounds of H records per half (as many rounds as the
    // larger of the two centres needs)
    float acc[NO2];
#pragma unroll
    for (int j = 0; j < NO2; ++j) acc[j] = 0.0f;
    const int cnt_a = ae - ab;
    const int rounds_to = max(cnt_a, __shfl_xor(cnt_a, H, kWave));
    for (int base = 0; base < rounds_to; base += H) {
        const int e = ab + base + hl;
        float *gl = gnL + hl * (na + 1);
        float *bl = bL + hl * (nlm + 1);
        if (e < ae) {
            float4 v = r.vec[e];
            int tj = types[r.nbr[e]];
            float f[KA] = {};
            chebyshev<KA>(v.w, t.rc_a, t.ka, f);
            const float *row = t.c_angular + size_t(ti * t.n_types + tj) * t.na * t.ka4;
            for (int n = 0; n < na; ++n) gl[n] = row_dot<KA>(row + n * t.ka4, t.ka4, f);
            float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
            const float ux = v.x * inv, uy = v.y * inv, uz = v.z * inv;
            int idx = 0;
            for (int L = 1; L <= t.l_max; ++L) {
                float wr = 1.0f, wi = 0.0f;   // (x + iy)^n1
                for (int n1 = 0; n1 <= L; ++n1) {
                    float zf, zfp;
                    zpoly(t, L, n1, uz, zf, zfp);
                    if (n1 == 0) {
                        bl[idx++] = zf;
                    } else {
                        next_w(ux, uy, wr, wi);
                        bl[idx++] = zf * wr;
                        bl[idx++] = zf * wi;
                    }
                }
            }
        }
        __syncthreads();
        const int cnt = max(0, min(H, cnt_a - base));
#pragma unroll
        for (int j = 0; j < NO2; ++j) {
            int o = hl + H * j;
            if (o >= nout) break;
            int n = o / nlm, c = o - n * nlm;
            float a = 0.0f;
            for (int k = 0; k < cnt; ++k) a += gnL[k * (na + 1) + n] * bL[k * (nlm + 1) + c];
            acc[j] += a;
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < NO2; ++j) {
        int o = hl + H * j;
        if (o >= nout) break;
        sL[o] = acc[j];
        if (valid) moments[size_t(i) * nout + o] = acc[j];
    }
    __syncthreads();
    if (valid) {
        float *out = q + size_t(i) * ldq + t.nr;
        for (int o = hl; o < na * t.num_L; o += H) {
            const int idx = o / na, n = o - idx * na;
            out[o] = invariant_one(t, sL + n * nlm, idx);
        }
    }
}

__device__ inline void zbl_pair(const ZblTables &z, int ti, int tj, float d, float &e,
                                float &de) {
    const float K = 14.399645f;
    float zi = z.z[ti], zj = z.z[tj];
    float a_inv = (z.zpow[ti] + z.zpow[tj]) * 2.134563f;
    float rin = z.rc_inner, rout = z.rc_outer;
    float co[8];
    for (int k = 0; k < 8; ++k) co[k] = z.universal[k];
    if (z.mode == RUNE_ZBL_FLEXIBLE) {
        int lo = min(ti, tj), hi = max(ti, tj);
        const float *p = z.pairs + size_t(lo * z.n_types - lo * (lo - 1) / 2 + hi - lo) * 10;
        rin = p[0];
        rout = p[1];
        for (int k = 0; k < 8; ++k) co[k] = p[2 + k];
    }
    float x = d * a_inv;
    float phi = 0.0f, dphi = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float ex = co[2 * k] * expf(-co[2 * k + 1] * x);
        phi += ex;
        dphi += -co[2 * k + 1] * a_inv * ex;
    }
    float pref = K * zi * zj;
    float scr = pref * phi / d;
    float dscr = pref * (dphi / d - phi / (d * d));
    float w = fmaxf(rout - rin, 1.0e-12f);
    float cut, dcut;
    if (d < rin) {
        cut = 1.0f;
        dcut = 0.0f;
    } else if (d < rout) {
        float a = kPi * (d - rin) / w;
        cut = 0.5f * cosf(a) + 0.5f;
        dcut = -0.5f * kPi / w * sinf(a);
    } else {
        cut = 0.0f;
        dcut = 0.0f;
    }
    e = 0.5f * scr * cut;
    de = 0.5f * (dscr * cut + scr * dcut);
}

// P centres per wave (P = 2: lanes 0-31 centre 2b, lanes 32-63 centre 2b + 1,
// for sparse lists on large grids, as k_descriptor_forward_pair).
template <int KR, int KA, int NA, bool kRegCubic = false, int P = 1>
__global__ void __launch_bounds__(kWave) k_descriptor_reverse(
    DescTables t, ZblTables z, Records r, const int32_t *types, const float *dq, int ldq,
    const float *moments, const float *dmom, const float4 *g_direct, float *energies,
    float4 *g, int want_grad) {
    extern __shared__ float lds[];
    constexpr int H = kWave / P;   // lanes per centre
    const int nlm = t.nlm, na = t.na, nout = na * nlm;
    const int half = P == 1 ? 0 : int(threadIdx.x) / H;
    const int lane = P == 1 ? int(threadIdx.x) : int(threadIdx.x) % H;
    const int i = P * int(blockIdx.x) + half;
    const bool valid = P == 1 || i < r.n_atoms;
    const int ic = P == 1 ? i : (valid ? i : r.n_atoms - 1);
    // per centre: dq row, moments, their weights, and a channel-major copy of
    // the weights, NA rows per channel (zero past na), 16-byte aligned: each
    // record reads a channel's weights with NA / 4 vector loads
    const int wt_off = (t.Q + 2 * nout + 3) & ~3;
    float *dqL = P == 1 ? lds : lds + half * (wt_off + NA * nlm);   // [Q]
    float *sL = dqL + t.Q;                           // [na*nlm]
    float *WL = sL + nout;                           // [na*nlm]
    float *WT = dqL + wt_off;                        // [nlm][NA]
    const int ti = types[ic];
    const int rb = r.view[4 * ic], re = r.view[4 * ic + 1];
    const int ab = r.view[4 * ic + 2], ae = r.view[4 * ic + 3];
    const int eb = r.ptr[ic], ee = valid ? r.ptr[ic + 1] : eb;
    if (want_grad) {
        for (int k = lane; k < t.Q; k += H) dqL[k] = dq[size_t(ic) * ldq + k];
        for (int o = lane; o < nout; o += H) {
            sL[o] = moments[size_t(ic) * nout + o];
            WL[o] = dmom ? dmom[size_t(ic) * nout + o] : 0.0f;
        }
        __syncthreads();
        invariant_gradient_all<kRegCubic, H>(t, sL, dqL + t.nr, WL, lane);
        __syncthreads();
        for (int o = lane; o < nlm * NA; o += H) {
            const int c = o / NA, n = o - c * NA;
            WT[o] = n < na ? WL[n * nlm + c] : 0.0f;
        }
        __syncthreads();
    }
    float zsum = 0.0f;
    for (int e = eb + lane; e < ee; e += H) {
        float4 v = r.vec[e];
        float d = v.w;
        float inv = 1.0f / fmaxf(d, 1.0e-12f);
        float ux = v.x * inv, uy = v.y * inv, uz = v.z * inv;
        int tj = types[r.nbr[e]];
        float gx = 0.0f, gy = 0.0f, gz = 0.0f;
        bool in_r = e >= rb && e < re;
        bool in_a = e >= ab && e < ae;
        if (want_grad && in_r) {
            float f[KR] = {}, fp[KR] = {};
            chebyshev_d<KR>(d, t.rc_r, t.kr, f, fp);
            const float *row = t.c_radial + size_t(ti * t.n_types + tj) * t.nr * t.kr4;
            float gs = 0.0f;
            for (int n = 0; n < t.nr; ++n) gs += dqL[n] * row_dot<KR>(row + n * t.kr4, t.kr4, fp);
            gx += gs * ux;
            gy += gs * uy;
            gz += gs * uz;
        }
        if (want_grad && in_a) {
            float f[KA] = {}, fp[KA] = {};
            chebyshev_d<KA>(d, t.rc_a, t.ka, f, fp);
            const float *row = t.c_angular + size_t(ti * t.n_types + tj) * t.na * t.ka4;
            float gn[NA], gnp[NA];
#pragma unroll
            for (int n = 0; n < NA; ++n) {
                float a = 0.0f, b = 0.0f;
                if (n < na) {
                    const float4 *r4 = reinterpret_cast<const float4 *>(row + n * t.ka4);
#pragma unroll
                    for (int q = 0; q < KA / 4; ++q) {
                        if (4 * q >= t.ka4) break;
                        const float4 c = r4[q];
                        a += c.x * f[4 * q];
                        b += c.x * fp[4 * q];
                        a += c.y * f[4 * q + 1];
                        b += c.y * fp[4 * q + 1];
                        a += c.z * f[4 * q + 2];
                        b += c.z * fp[4 * q + 2];
                        a += c.w * f[4 * q + 3];
                        b += c.w * fp[4 * q + 3];
                    }
                }
                gn[n] = a;
                gnp[n] = b;
            }
            float rs = 0.0f, dx = 0.0f, dy = 0.0f, dz = 0.0f, proj = 0.0f;
            int c = 0;
            // one angular channel c with basis value b and gradient (bx, by, bz)
            auto channel = [&](float b, float bx, float by, float bz) {
                float wsum = 0.0f, wsump = 0.0f;
                const float4 *w4 = reinterpret_cast<const float4 *>(WT + c * NA);
#pragma unroll
                for (int q = 0; q < NA / 4; ++q) {
                    const float4 w = w4[q];
                    wsum += w.x * gn[4 * q];
                    wsump += w.x * gnp[4 * q];
                    wsum += w.y * gn[4 * q + 1];
                    wsump += w.y * gnp[4 * q + 1];
                    wsum += w.z * gn[4 * q + 2];
                    wsump += w.z * gnp[4 * q + 2];
                    wsum += w.w * gn[4 * q + 3];
                    wsump += w.w * gnp[4 * q + 3];
                }
                rs += wsump * b;
                dx += wsum * bx;
                dy += wsum * by;
                dz += wsum * bz;
                proj += wsum * (ux * bx + uy * by + uz * bz);
                ++c;
            };
            for (int L = 1; L <= t.l_max; ++L) {
                float wr = 1.0f, wi = 0.0f;   // (x + iy)^n1
                for (int n1 = 0; n1 <= L; ++n1) {
                    float zf, zfp;
                    zpoly(t, L, n1, uz, zf, zfp);
                    if (n1 == 0) {
                        channel(zf, 0.0f, 0.0f, zfp);
                    } else {
                        const float pr = wr, pi = wi;   // (x + iy)^(n1-1)
                        next_w(ux, uy, wr, wi);
                        const float zn = zf * float(n1);
                        channel(zf * wr, zn * pr, -zn * pi, zfp * wr);
                        channel(zf * wi, zn * pi, zn * pr, zfp * wi);
                    }
                }
            }
            gx += rs * ux + (dx - proj * ux) * inv;
            gy += rs * uy + (dy - proj * uy) * inv;
            gz += rs * uz + (dz - proj * uz) * inv;
        }
        bool in_z = z.mode != RUNE_ZBL_NONE && (z.on_angular ? in_a : in_r);
        if (in_z) {
            float ez, dez;
            zbl_pair(z, ti, tj, fmaxf(d, 1.0e-12f), ez, dez);
            zsum += ez;
            gx += dez * ux;
            gy += dez * uy;
            gz += dez * uz;
        }
        if (want_grad) {
            if (g_direct) {
                float4 gd = g_direct[e];
                gx += gd.x;
                gy += gd.y;
                gz += gd.z;
            }
            g[e] = make_float4(gx, gy, gz, 0.0f);
        }
    }
    if (z.mode != RUNE_ZBL_NONE) {
        float s = zsum;
#pragma unroll
        for (int off = H / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, kWave);
        if (lane == 0 && valid) energies[i] += s;
    }
}

// ---- any channel count and basis size ----
// The kernels above keep a lane's basis values (<= kMaxKr / kMaxKa) and
// channel values (<= kMaxNr / kMaxNa) in registers.  These variants give
// each lane LDS rows for them instead, so every model the reference accepts
// (any n_max, basis_size) evaluates; same wave-per-centre structure, same
// fixed summation order per output.

// f_k(r) (and f'_k(r) when fp) for k < k_max into one lane's LDS row.
__device__ inline void chebyshev_row(float r, float rc, int k_max, float *f, float *fp) {
    const float rcinv = 1.0f / rc;
    const float arg = kPi * r * rcinv;
    const float fc = 0.5f * cosf(arg) + 0.5f;
    const float fcp = -0.5f * kPi * rcinv * sinf(arg);
    const float rs = r * rcinv - 1.0f;
    const float x = 2.0f * rs * rs - 1.0f;
    const float dxdr = 4.0f * rs * rcinv;
    f[0] = fc;
    if (fp) fp[0] = fcp;
    float t2 = 1.0f, t1 = x, u2 = 1.0f, u1 = 2.0f * x;
    for (int k = 1; k < k_max; ++k) {
        if (k == 1) {
            const float core = 0.5f * (x + 1.0f);
            f[1] = core * fc;
            if (fp) fp[1] = 0.5f * dxdr * fc + core * fcp;
        } else {
            const float tn = 2.0f * x * t1 - t2, un = 2.0f * x * u1 - u2;
            const float core = 0.5f * (tn + 1.0f);
            f[k] = core * fc;
            if (fp) fp[k] = 0.5f * float(k) * u1 * dxdr * fc + core * fcp;
            t2 = t1;
            t1 = tn;
            u2 = u1;
            u1 = un;
        }
    }
}

// Output chunk of the moment accumulators of the wide forward kernel.
constexpr int kWideOut = 16;

__global__ void __launch_bounds__(kWave) k_descriptor_forward_wide(DescTables t, Records r,
                                                                   const int32_t *types, float *q,
                                                                   int ldq, float *moments) {
    extern __shared__ float lds[];
    const int nlm = t.nlm, na = t.na, nout = na * nlm, kmax = max(t.kr, t.ka);
    float *fL = lds;                                // [64][kmax + 1] basis rows
    float *gnL = fL + kWave * (kmax + 1);           // [64][na + 1]
    float *bL = gnL + kWave * (na + 1);             // [64][nlm + 1]
    float *sL = bL + kWave * (nlm + 1);             // [na * nlm]
    const int i = blockIdx.x, lane = threadIdx.x;
    const int ti = types[i];
    const int rb = r.view[4 * i], re = r.view[4 * i + 1];
    const int ab = r.view[4 * i + 2], ae = r.view[4 * i + 3];
    float *f = fL + lane * (kmax + 1);
    // radial channels, 16 at a time (the basis rows are rebuilt per group)
    for (int n0 = 0; n0 < t.nr; n0 += 16) {
        float qr[16];
#pragma unroll
        for (int n = 0; n < 16; ++n) qr[n] = 0.0f;
        for (int e = rb + lane; e < re; e += kWave) {
            const float4 v = r.vec[e];
            const int tj = types[r.nbr[e]];
            chebyshev_row(v.w, t.rc_r, t.kr, f, nullptr);
            const float *row = t.c_radial + size_t(ti * t.n_types + tj) * t.nr * t.kr4;
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                if (n0 + n >= t.nr) break;
                const float *cr = row + (n0 + n) * t.kr4;
                float a = 0.0f;
                for (int k = 0; k < t.kr; ++k) a += cr[k] * f[k];
                qr[n] += a;
            }
        }
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            if (n0 + n >= t.nr) break;
            const float v = wave_sum(qr[n]);
            if (lane == 0) q[size_t(i) * ldq + n0 + n] = v;
        }
    }
    // angular moments s[n][lm] = sum_e gn[e][n] b[e][lm], outputs in chunks
    for (int o0 = 0; o0 < nout; o0 += kWideOut * kWave) {
        float acc[kWideOut];
#pragma unroll
        for (int j = 0; j < kWideOut; ++j) acc[j] = 0.0f;
        for (int base = ab; base < ae; base += kWave) {
            const int e = base + lane;
            float *gl = gnL + lane * (na + 1);
            float *bl = bL + lane * (nlm + 1);
            if (e < ae) {
                const float4 v = r.vec[e];
                const int tj = types[r.nbr[e]];
                chebyshev_row(v.w, t.rc_a, t.ka, f, nullptr);
                const float *row = t.c_angular + size_t(ti * t.n_types + tj) * t.na * t.ka4;
                for (int n = 0; n < na; ++n) {
                    const float *cr = row + n * t.ka4;
                    float a = 0.0f;
                    for (int k = 0; k < t.ka; ++k) a += cr[k] * f[k];
                    gl[n] = a;
                }
                const float inv = 1.0f / fmaxf(v.w, 1.0e-12f);
                const float ux = v.x * inv, uy = v.y * inv, uz = v.z * inv;
                int idx = 0;
                for (int L = 1; L <= t.l_max; ++L) {
                    float wr = 1.0f, wi = 0.0f;
                    for (int n1 = 0; n1 <= L; ++n1) {
                        float zf, zfp;
                        zpoly(t, L, n1, uz, zf, zfp);
                        if (n1 == 0) {
                            bl[idx++] = zf;
                        } else {
                            next_w(ux, uy, wr, wi);
                            bl[idx++] = zf * wr;
                            bl[idx++] = zf * wi;
                        }
                    }
                }
            } else {
                for (int n = 0; n < na; ++n) gl[n] = 0.0f;
                for (int c = 0; c < nlm; ++c) bl[c] = 0.0f;
            }
            __syncthreads();
            const int cnt = min(kWave, ae - base);
#pragma unroll
            for (int j = 0; j < kWideOut; ++j) {
                const int o = o0 + lane + kWave * j;
                if (o >= nout) break;
                const int n = o / nlm, c = o - n * nlm;
                float a = 0.0f;
                for (int k = 0; k < cnt; ++k) a += gnL[k * (na + 1) + n] * bL[k * (nlm + 1) + c];
                acc[j] += a;
            }
            __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < kWideOut; ++j) {
            const int o = o0 + lane + kWave * j;
            if (o >= nout) break;
            sL[o] = acc[j];
            moments[size_t(i) * nout + o] = acc[j];
        }
    }
    __syncthreads();
    invariants_all(t, sL, q + size_t(i) * ldq + t.nr, lane);
}

__global__ void __launch_bounds__(kWave) k_descriptor_reverse_wide(
    DescTables t, ZblTables z, Records r, const int32_t *types, const float *dq, int ldq,
    const float *moments, const float *dmom, const float4 *g_direct, float *energies,
    float4 *g, int want_grad) {
    extern __shared__ float lds[];
    const int nlm = t.nlm, na = t.na, nout = na * nlm, kmax = max(t.kr, t.ka);
    float *dqL = lds;                                   // [Q]
    float *sL = dqL + t.Q;                              // [na * nlm]
    float *WL = sL + nout;                              // [na * nlm]
    float *fL = WL + nout;                              // [64][kmax + 1]
    float *fpL = fL + kWave * (kmax + 1);               // [64][kmax + 1]
    float *gnL = fpL + kWave * (kmax + 1);              // [64][na + 1]
    float *gnpL = gnL + kWave * (na + 1);               // [64][na + 1]
    const int i = blockIdx.x, lane = threadIdx.x;
    const int ti = types[i];
    const int rb = r.view[4 * i], re = r.view[4 * i + 1];
    const int ab = r.view[4 * i + 2], ae = r.view[4 * i + 3];
    const int eb = r.ptr[i], ee = r.ptr[i + 1];
    if (want_grad) {
        for (int k = lane; k < t.Q; k += kWave) dqL[k] = dq[size_t(i) * ldq + k];
        for (int o = lane; o < nout; o += kWave) {
            sL[o] = moments[size_t(i) * nout + o];
            WL[o] = dmom ? dmom[size_t(i) * nout + o] : 0.0f;
        }
        __syncthreads();
        invariant_gradient_all(t, sL, dqL + t.nr, WL, lane);
        __syncthreads();
    }
    float *f = fL + lane * (kmax + 1), *fp = fpL + lane * (kmax + 1);
    float *gn = gnL + lane * (na + 1), *gnp = gnpL + lane * (na + 1);
    float zsum = 0.0f;
    for (int e = eb + lane; e < ee; e += kWave) {
        const float4 v = r.vec[e];
        const float d = v.w;
        const float inv = 1.0f / fmaxf(d, 1.0e-12f);
        const float ux = v.x * inv, uy = v.y * inv, uz = v.z * inv;
        const int tj = types[r.nbr[e]];
        float gx = 0.0f, gy = 0.0f, gz = 0.0f;
        const bool in_r = e >= rb && e < re;
        const bool in_a = e >= ab && e < ae;
        if (want_grad && in_r) {
            chebyshev_row(d, t.rc_r, t.kr, f, fp);
            const float *row = t.c_radial + size_t(ti * t.n_types + tj) * t.nr * t.kr4;
            float gs = 0.0f;
            for (int n = 0; n < t.nr; ++n) {
                const float *cr = row + n * t.kr4;
                float a = 0.0f;
                for (int k = 0; k < t.kr; ++k) a += cr[k] * fp[k];
                gs += dqL[n] * a;
            }
            gx += gs * ux;
            gy += gs * uy;
            gz += gs * uz;
        }
        if (want_grad && in_a) {
            chebyshev_row(d, t.rc_a, t.ka, f, fp);
            const float *row = t.c_angular + size_t(ti * t.n_types + tj) * t.na * t.ka4;
            for (int n = 0; n < na; ++n) {
                const float *cr = row + n * t.ka4;
                float a = 0.0f, b = 0.0f;
                for (int k = 0; k < t.ka; ++k) {
                    a += cr[k] * f[k];
                    b += cr[k] * fp[k];
                }
                gn[n] = a;
                gnp[n] = b;
            }
            float rs = 0.0f, dx = 0.0f, dy = 0.0f, dz = 0.0f, proj = 0.0f;
            int c = 0;
            auto channel = [&](float b, float bx, float by, float bz) {
                float wsum = 0.0f, wsump = 0.0f;
                for (int n = 0; n < na; ++n) {
                    const float w = WL[n * nlm + c];
                    wsum += w * gn[n];
                    wsump += w * gnp[n];
                }
                rs += wsump * b;
                dx += wsum * bx;
                dy += wsum * by;
                dz += wsum * bz;
                proj += wsum * (ux * bx + uy * by + uz * bz);
                ++c;
            };
            for (int L = 1; L <= t.l_max; ++L) {
                float wr = 1.0f, wi = 0.0f;
                for (int n1 = 0; n1 <= L; ++n1) {
                    float zf, zfp;
                    zpoly(t, L, n1, uz, zf, zfp);
                    if (n1 == 0) {
                        channel(zf, 0.0f, 0.0f, zfp);
                    } else {
                        const float pr = wr, pi = wi;
                        next_w(ux, uy, wr, wi);
                        const float zn = zf * float(n1);
                        channel(zf * wr, zn * pr, -zn * pi, zfp * wr);
                        channel(zf * wi, zn * pi, zn * pr, zfp * wi);
                    }
                }
            }
            gx += rs * ux + (dx - proj * ux) * inv;
            gy += rs * uy + (dy - proj * uy) * inv;
            gz += rs * uz + (dz - proj * uz) * inv;
        }
        const bool in_z = z.mode != RUNE_ZBL_NONE && (z.on_angular ? in_a : in_r);
        if (in_z) {
            float ez, dez;
            zbl_pair(z, ti, tj, fmaxf(d, 1.0e-12f), ez, dez);
            zsum += ez;
            gx += dez * ux;
            gy += dez * uy;
            gz += dez * uz;
        }
        if (want_grad) {
            if (g_direct) {
                const float4 gd = g_direct[e];
                gx += gd.x;
                gy += gd.y;
                gz += gd.z;
            }
            g[e] = make_float4(gx, gy, gz, 0.0f);
        }
    }
    if (z.mode != RUNE_ZBL_NONE) {
        const float sz = wave_sum(zsum);
        if (lane == 0) energies[i] += sz;
    }
}

// The register kernels cover these sizes; larger ones take the wide kernels.
bool descriptor_fits_registers(const DescTables &t) {
    return t.nr <= kMaxNr && t.na <= kMaxNa && t.kr <= kMaxKr && t.ka <= kMaxKa;
}

// Compact register arrays (basis 20 / 16, 12 angular channels, 5 moment
// outputs per lane: 67 / 90 VGPRs for the forward / reverse kernel instead
// of 140 / 145, so 7 / 5 waves per SIMD instead of 3) for the models that
// fit them, the OAM and NEP models among them.
constexpr int kCompactKr = 20, kCompactKa = 16, kCompactNa = 12, kCompactOut = 5;
// Up to this many centres (a few waves per SIMD at most) the reverse kernel
// keeps the cubic-invariant gradients in registers: its wave latency is the
// kernel time there, and the extra registers cost nothing.
constexpr int kSmallDescAtoms = 8192;
// From this many centres (more than one round of one-centre waves) a sparse
// list takes the two-centres-per-wave kernels.
constexpr int kPairDescAtoms = 8192;
bool descriptor_compact(const DescTables &t) {
    return t.nr <= kMaxNr && t.kr <= kCompactKr && t.ka <= kCompactKa && t.na <= kCompactNa &&
           t.na * t.nlm <= kCompactOut * kWave;
}

}  // namespace

static void allow_lds(const void *kernel, size_t lds) {
    if (lds > 65536)
        RUNE_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           int(lds)));
}

void descriptor_forward(const DescTables &t, const Records &r, int64_t n_records,
                        const int32_t *types, float *q, int ldq, float *moments, hipStream_t s) {
    if (r.n_atoms == 0) return;
    if (!descriptor_fits_registers(t)) {
        const int kmax = std::max(t.kr, t.ka);
        const size_t lds = sizeof(float) * (kWave * (kmax + 1) + kWave * (t.na + 1) +
                                             kWave * (t.nlm + 1) + t.na * t.nlm);
        allow_lds(reinterpret_cast<const void *>(&k_descriptor_forward_wide), lds);
        hipLaunchKernelGGL(k_descriptor_forward_wide, dim3(r.n_atoms), dim3(kWave), lds, s, t, r,
                           types, q, ldq, moments);
        RUNE_HIP_CHECK(hipGetLastError());
        return;
    }
    // LDS rows for `ch` angular records per round (the moment row reuses
    // them afterwards).  Half-wave rounds halve the LDS of a block, so twice
    // as many blocks fit a CU; they pay when a centre has at most 32 angular
    // records, estimated from the mean record count and the cutoff volumes.
    const double ratio = t.rc_a < t.rc_r ? double(t.rc_a) / t.rc_r : 1.0;
    const double ang = double(n_records) / r.n_atoms * ratio * ratio * ratio;
    const int ch = descriptor_compact(t) && ang <= 32.0 ? 32 : kWave;
    const size_t lds = sizeof(float) * std::max<size_t>(size_t(ch) * (t.na + t.nlm + 2),
                                                        size_t(t.na) * t.nlm);
    // sparse lists on grids of more than one round of waves: two centres per
    // wave (rounds of 32 records per half)
    const double mean = double(n_records) / r.n_atoms;
    if (descriptor_compact(t) && mean <= 32.0 && r.n_atoms >= kPairDescAtoms) {
        const size_t hstride = std::max<size_t>(size_t(kWave / 2) * (t.na + t.nlm + 2),
                                                size_t(t.na) * t.nlm);
        const dim3 grid((r.n_atoms + 1) / 2);
        const size_t plds = sizeof(float) * 2 * hstride;
        if (t.na * t.nlm <= kCompactOut * kWave / 2)   // moments per half-lane
            hipLaunchKernelGGL((k_descriptor_forward_pair<kCompactKr, kCompactKa, kMaxNr,
                                                          kCompactOut>),
                               grid, dim3(kWave), plds, s, t, r, types, q, ldq, moments);
        else
            hipLaunchKernelGGL((k_descriptor_forward_pair<kCompactKr, kCompactKa, kMaxNr,
                                                          2 * kCompactOut>),
                               grid, dim3(kWave), plds, s, t, r, types, q, ldq, moments);
    } else if (descriptor_compact(t) && t.nlm <= 32 && ch == 32)
        hipLaunchKernelGGL((k_descriptor_forward<kCompactKr, kCompactKa, kMaxNr, kCompactOut, 32,
                                                 true>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, r, types, q, ldq, moments);
    else if (descriptor_compact(t) && t.nlm <= 32)
        hipLaunchKernelGGL((k_descriptor_forward<kCompactKr, kCompactKa, kMaxNr, kCompactOut,
                                                 kWave, true>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, r, types, q, ldq, moments);
    else if (descriptor_compact(t) && ch == 32)
        hipLaunchKernelGGL((k_descriptor_forward<kCompactKr, kCompactKa, kMaxNr, kCompactOut, 32>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, r, types, q, ldq, moments);
    else if (descriptor_compact(t))
        hipLaunchKernelGGL((k_descriptor_forward<kCompactKr, kCompactKa, kMaxNr, kCompactOut>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, r, types, q, ldq, moments);
    else
        hipLaunchKernelGGL((k_descriptor_forward<kMaxKr, kMaxKa, kMaxNr,
                                                 (kMaxNa * kMaxLm + kWave - 1) / kWave>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, r, types, q, ldq, moments);
    RUNE_HIP_CHECK(hipGetLastError());
}

void descriptor_reverse(const DescTables &t, const ZblTables &z, const Records &r,
                        int64_t n_records, const int32_t *types, const float *dq, int ldq,
                        const float *moments, const float *dmom, const float4 *g_direct,
                        float *energies, float4 *g, int want_grad, hipStream_t s) {
    if (r.n_atoms == 0) return;
    if (!want_grad && z.mode == RUNE_ZBL_NONE) return;
    if (!descriptor_fits_registers(t)) {
        const int kmax = std::max(t.kr, t.ka);
        const size_t lds = sizeof(float) * (t.Q + 2 * t.na * t.nlm + 2 * kWave * (kmax + 1) +
                                             2 * kWave * (t.na + 1));
        allow_lds(reinterpret_cast<const void *>(&k_descriptor_reverse_wide), lds);
        hipLaunchKernelGGL(k_descriptor_reverse_wide, dim3(r.n_atoms), dim3(kWave), lds, s, t, z,
                           r, types, dq, ldq, moments, dmom, g_direct, energies, g, want_grad);
        RUNE_HIP_CHECK(hipGetLastError());
        return;
    }
    static_assert(kCompactNa % 4 == 0 && kMaxNa % 4 == 0, "channel-major rows of 4-float vectors");
    const int na_pad = descriptor_compact(t) ? kCompactNa : kMaxNa;
    const size_t lds = sizeof(float) * (((t.Q + 2 * t.na * t.nlm + 3) & ~3) + size_t(na_pad) * t.nlm);
    const double mean = double(n_records) / r.n_atoms;
    if (descriptor_compact(t) && mean <= 32.0 && r.n_atoms >= kPairDescAtoms)
        hipLaunchKernelGGL((k_descriptor_reverse<kCompactKr, kCompactKa, kCompactNa, false, 2>),
                           dim3((r.n_atoms + 1) / 2), dim3(kWave), 2 * lds, s, t, z, r, types, dq,
                           ldq, moments, dmom, g_direct, energies, g, want_grad);
    else if (descriptor_compact(t) && r.n_atoms <= kSmallDescAtoms)
        hipLaunchKernelGGL((k_descriptor_reverse<kCompactKr, kCompactKa, kCompactNa, true>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, z, r, types, dq, ldq, moments,
                           dmom, g_direct, energies, g, want_grad);
    else if (descriptor_compact(t))
        hipLaunchKernelGGL((k_descriptor_reverse<kCompactKr, kCompactKa, kCompactNa>),
                           dim3(r.n_atoms), dim3(kWave), lds, s, t, z, r, types, dq, ldq, moments,
                           dmom, g_direct, energies, g, want_grad);
    else
        hipLaunchKernelGGL((k_descriptor_reverse<kMaxKr, kMaxKa, kMaxNa>), dim3(r.n_atoms),
                           dim3(kWave), lds, s, t, z, r, types, dq, ldq, moments, dmom, g_direct,
                           energies, g, want_grad);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
