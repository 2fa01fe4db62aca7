// K1: canonical periodic neighbour lists (cell-list binning, exact fp64 test).
//
// Semantics follow rune/mobius/interface/batch.py:42-102: every image pair
// (i, j, S) with (p_j + S.cell) - p_i shorter than the cutoff, self pairs at
// S = 0 excluded, radial and angular membership decided in fp64 by
//     o_d = (S0*c0d + S1*c1d) + S2*c2d,   v = (p_j + o) - p_i,
//     d2  = (v0*v0 + v1*v1) + v2*v2 < rc*rc
// with no fused multiply-add, so the edge set is reproducible bit for bit.
// Binning only proposes candidates; it never decides membership.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>

#include <type_traits>

#include "nlist.hpp"

#pragma clang fp contract(off)

namespace rune {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;

struct Geo {
    double cell[9];     // rows = lattice vectors
    double inv[9];      // inverse of cell (frac = p . inv)
    int pbc[3];
    int nb[3];          // periodic directions: bins per cell period
    double bs[3];       // bins per unit of fractional coordinate (nb when periodic)
    double lo[3];       // open directions: lowest bin index holding an atom (0 otherwise)
    int nbin[3];        // bins in use per direction (nb for periodic directions)
    int m[3];           // stencil reach per direction
    int bin_offset;     // first global bin of this structure
    int atom_begin, atom_end;
};

__device__ inline int find_structure(const int32_t *sptr, int nstruct, int atom) {
    int lo = 0, hi = nstruct - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (sptr[mid] <= atom) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ inline void frac_of(const Geo &g, const double *p, double *f) {
    for (int d = 0; d < 3; ++d)
        f[d] = (p[0] * g.inv[0 * 3 + d] + p[1] * g.inv[1 * 3 + d]) + p[2] * g.inv[2 * 3 + d];
}

__global__ void bin_atoms(int n, const double *pos, const int32_t *sptr, int nstruct,
                          const Geo *geo, int32_t *atom_bin, int32_t *atom_wrap,
                          int32_t *atom_cell, int32_t *bin_count) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int s = find_structure(sptr, nstruct, i);
    const Geo &g = geo[s];
    double f[3];
    frac_of(g, pos + 3 * i, f);
    int b[3], w[3];
    for (int d = 0; d < 3; ++d) {
        double fd = f[d];
        w[d] = 0;
        if (g.pbc[d]) {
            double fl = floor(fd);
            w[d] = int(fl);
            fd -= fl;
        }
        // open directions: bins from the lowest one holding an atom, so no
        // atom is clamped into an edge bin (the clamp is only a safety net)
        double x = floor(fd * g.bs[d]) - g.lo[d];
        x = fmin(fmax(x, 0.0), double(g.nbin[d] - 1));
        b[d] = int(x);
    }
    int flat = g.bin_offset + (b[0] * g.nbin[1] + b[1]) * g.nbin[2] + b[2];
    atom_bin[i] = flat;
    atom_wrap[3 * i + 0] = w[0];
    atom_wrap[3 * i + 1] = w[1];
    atom_wrap[3 * i + 2] = w[2];
    atom_cell[3 * i + 0] = b[0];
    atom_cell[3 * i + 1] = b[1];
    atom_cell[3 * i + 2] = b[2];
    atomicAdd(bin_count + flat, 1);
}

__global__ void fill_bins(int n, const int32_t *atom_bin, const int32_t *bin_start,
                          int32_t *bin_cursor, int32_t *bin_atoms) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int b = atom_bin[i];
    int slot = atomicAdd(bin_cursor + b, 1);
    bin_atoms[bin_start[b] + slot] = i;
}

// Order-preserving map of a double to 64 bits (for integer atomic min / max).
__device__ inline unsigned long long ordered_bits(double x) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(x);
    return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// Extent of each structure's fractional coordinates along its open
// (non-periodic) directions: ext[3 s + d] = min, ext[3 (nstruct + s) + d] =
// max, as ordered bits (min entries start all ones, max entries zero).  Lanes past
// the end stand in for the last atom (min / max are idempotent); a wave whose
// lanes share one structure combines them before its atomics.
__global__ void frac_extent(int n, const double *pos, const int32_t *sptr, int nstruct,
                            const Geo *geo, unsigned long long *ext) {
    const int i = min(int(blockIdx.x * blockDim.x + threadIdx.x), n - 1);
    const int s = find_structure(sptr, nstruct, i);
    const Geo &g = geo[s];
    double f[3];
    frac_of(g, pos + 3 * i, f);
    double lo[3] = {f[0], f[1], f[2]}, hi[3] = {f[0], f[1], f[2]};
    const bool uniform = __all(s == __shfl(s, 0)) != 0;
    if (uniform) {
        for (int off = 32; off > 0; off >>= 1)
            for (int d = 0; d < 3; ++d) {
                lo[d] = fmin(lo[d], __shfl_xor(lo[d], off));
                hi[d] = fmax(hi[d], __shfl_xor(hi[d], off));
            }
    }
    if (uniform && (threadIdx.x & 63) != 0) return;
    for (int d = 0; d < 3; ++d) {
        if (g.pbc[d]) continue;
        atomicMin(ext + 3 * s + d, ordered_bits(lo[d]));
        atomicMax(ext + 3 * (nstruct + s) + d, ordered_bits(hi[d]));
    }
}

// Atoms listed bin by bin in the rank order perm (bins of all structures):
// rank_count[r] = atoms of bin perm[r], then (after a scan) the copy.
__global__ void rank_counts(int nbins, const int32_t *perm, const int32_t *bin_count,
                            int32_t *rank_count) {
    int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < nbins) rank_count[r] = bin_count[perm[r]];
}

__global__ void order_atoms(int nbins, const int32_t *perm, const int32_t *bin_start,
                            const int32_t *bin_count, const int32_t *rank_start,
                            const int32_t *bin_atoms, int32_t *order) {
    int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= nbins) return;
    const int b = perm[r], src = bin_start[b], dst = rank_start[r];
    for (int q = 0; q < bin_count[b]; ++q) order[dst + q] = bin_atoms[src + q];
}

// Exact fp64 squared distance of image (j, S) seen from i.
__device__ inline double pair_d2(const double *pos, const Geo &g, int i, int j, const int *S,
                                 double *v) {
    double r2 = 0.0;
    for (int d = 0; d < 3; ++d) {
        double o = (double(S[0]) * g.cell[0 * 3 + d] + double(S[1]) * g.cell[1 * 3 + d]) +
                   double(S[2]) * g.cell[2 * 3 + d];
        v[d] = (pos[3 * j + d] + o) - pos[3 * i + d];
    }
    r2 = (v[0] * v[0] + v[1] * v[1]) + v[2] * v[2];
    return r2;
}

// Record keys.  A 64-bit key holds the class (bits 62-63), the neighbour
// index j (bits 32-61; atom counts are below 2^30) and the image shift S as
// three 10-bit fields offset by kShiftBias (bits 20-29, 10-19, 0-9), so
// ascending keys order a centre's records by (class, j, S0, S1, S2).  A shift
// outside [-kShiftBias, kShiftBias) (an atom more than 511 periods from the
// cell) has no key: the builder reports it instead of aliasing it.
constexpr int kShiftBias = 512;

__device__ inline bool shift_fits(const int *S) {
    bool ok = true;
    for (int d = 0; d < 3; ++d) ok = ok && S[d] >= -kShiftBias && S[d] < kShiftBias;
    return ok;
}

__device__ inline uint64_t make_key(int cls, int j, const int *S) {
    uint64_t k = uint64_t(cls) << 62;
    k |= uint64_t(uint32_t(j)) << 32;
    k |= uint64_t(uint32_t(S[0] + kShiftBias) & 0x3ff) << 20;
    k |= uint64_t(uint32_t(S[1] + kShiftBias) & 0x3ff) << 10;
    k |= uint64_t(uint32_t(S[2] + kShiftBias) & 0x3ff);
    return k;
}

__device__ inline int key_neighbor(uint64_t key) { return int((key >> 32) & 0x3fffffffull); }

__device__ inline void key_shift(uint64_t key, int *S) {
    S[0] = int((key >> 20) & 0x3ff) - kShiftBias;
    S[1] = int((key >> 10) & 0x3ff) - kShiftBias;
    S[2] = int(key & 0x3ff) - kShiftBias;
}

// Candidate enumeration, one atom per wave, in one pass: the stencil cells
// (bins within the stencil reach, periodic images by wrapping) are taken 64
// at a time, a wave scan of their sizes flattens their candidates into one
// index range, and the 64 lanes test 64 candidates at a time with the exact
// fp64 test.  Ballots count the members (union, radial, angular) and give
// each its slot in the atom's row of `keys` ([n, cap], cap = the larger
// neighbour limit, so a centre within the limits always fits).  The centre's
// keys are then sorted by rank in LDS (each key's rank is the number of
// smaller keys; keys of one centre are distinct, since each (j, S) image is
// proposed once); centres with more than kWaveKeys keys fall back to lane
// 0's insertion sort in global memory.
constexpr int kWaveKeys = 1024;

// LDS keys per wave for rows of at most `cap` keys (the neighbour limit):
// rows that cannot exceed 128 or 256 keys take the smaller arrays, which
// keeps more waves resident per CU; launch(std::integral_constant<int, KW>).
template <typename F>
void by_key_lds(int cap, F &&launch) {
    if (cap <= 128)
        launch(std::integral_constant<int, 128>{});
    else if (cap <= 256)
        launch(std::integral_constant<int, 256>{});
    else
        launch(std::integral_constant<int, kWaveKeys>{});
}

__device__ inline void wave_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Counts of centre i (and the overflow flag), then its keys sorted ascending:
// by rank in LDS when they all fit there (kl holds the first KW keys),
// else by lane 0's insertion sort in global memory.
template <int KW>
__device__ inline void finish_centre(int i, int lane, int cu, int cr, int ca, int max_r, int max_a,
                                     int cap, const uint64_t *kl, uint64_t *out,
                                     int32_t *cnt_union, int32_t *cnt_r, int32_t *cnt_a,
                                     int32_t *error_flag) {
    if (lane == 0) {
        cnt_union[i] = cu;
        cnt_r[i] = cr;
        cnt_a[i] = ca;
        if (cr > max_r || ca > max_a || cu > cap) atomicOr(error_flag, 1);
    }
    if (cu > cap) return;
    if (cu <= KW) {
        for (int a = lane; a < cu; a += kWave) {
            const uint64_t x = kl[a];
            int rank = 0;
            for (int b = 0; b < cu; ++b) rank += kl[b] < x ? 1 : 0;
            out[rank] = x;
        }
        return;
    }
    // insertion sort of this centre's keys: (class, j, S) ascending
    if (lane != 0) return;
    for (int a = 1; a < cu; ++a) {
        const uint64_t x = out[a];
        int b = a - 1;
        while (b >= 0 && out[b] > x) {
            out[b + 1] = out[b];
            --b;
        }
        out[b + 1] = x;
    }
}

template <int KW>
__global__ void __launch_bounds__(256) enumerate_flat(
    int n, const double *pos, const int32_t *sptr, int nstruct, const Geo *geo,
    const int32_t *atom_wrap, const int32_t *atom_cell, const int32_t *bin_start,
    const int32_t *bin_atoms, double rc2_r, double rc2_a, double rc2_max, int max_r, int max_a,
    int cap, int32_t *cnt_union, int32_t *cnt_r, int32_t *cnt_a, int32_t *error_flag,
    uint64_t *keys) {
    __shared__ uint64_t kl[4][KW];
    __shared__ int cst[4][kWave], cbg[4][kWave], cT[4][kWave][3];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + wave;
    if (i >= n) return;
    const int s = find_structure(sptr, nstruct, i);
    const Geo &g = geo[s];
    const int wi[3] = {atom_wrap[3 * i], atom_wrap[3 * i + 1], atom_wrap[3 * i + 2]};
    const int ci[3] = {atom_cell[3 * i], atom_cell[3 * i + 1], atom_cell[3 * i + 2]};
    const int sx = 2 * g.m[0] + 1, sy = 2 * g.m[1] + 1, sz = 2 * g.m[2] + 1;
    const int ncell = sx * sy * sz;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint64_t *out = keys + size_t(i) * cap;
    int cu = 0, cr = 0, ca = 0;
    for (int c0 = 0; c0 < ncell; c0 += kWave) {
        const int c = c0 + lane;
        int cnt = 0, beg = 0, T[3] = {0, 0, 0};
        if (c < ncell) {
            const int dd[3] = {c / (sz * sy) - g.m[0], (c / sz) % sy - g.m[1], c % sz - g.m[2]};
            int bb[3];
            bool ok = true;
            for (int d = 0; d < 3; ++d) {
                const int b = ci[d] + dd[d];
                if (g.pbc[d]) {
                    const int t = (b >= 0) ? b / g.nb[d] : -((-b + g.nb[d] - 1) / g.nb[d]);
                    T[d] = t;
                    bb[d] = b - t * g.nb[d];
                } else {
                    bb[d] = b;
                    ok = ok && (b >= 0 && b < g.nbin[d]);
                }
            }
            if (ok) {
                const int flat = g.bin_offset + (bb[0] * g.nbin[1] + bb[1]) * g.nbin[2] + bb[2];
                beg = bin_start[flat];
                cnt = bin_start[flat + 1] - beg;
            }
        }
        int incl = cnt;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int v = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += v;
        }
        const int total = __shfl(incl, kWave - 1, kWave);
        wave_fence();
        cst[wave][lane] = incl - cnt;
        cbg[wave][lane] = beg;
        cT[wave][lane][0] = T[0];
        cT[wave][lane][1] = T[1];
        cT[wave][lane][2] = T[2];
        wave_fence();
        for (int t0 = 0; t0 < total; t0 += kWave) {
            const int t = t0 + lane;
            bool pass = false, in_r = false, in_a = false;
            int j = 0, S[3] = {0, 0, 0};
            if (t < total) {
                // the cell holding candidate t: the last one starting at or before t
                int lo = 0, hi = kWave - 1;
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (cst[wave][mid] <= t) lo = mid; else hi = mid - 1;
                }
                j = bin_atoms[cbg[wave][lo] + (t - cst[wave][lo])];
                for (int d = 0; d < 3; ++d)
                    S[d] = g.pbc[d] ? (cT[wave][lo][d] - atom_wrap[3 * j + d] + wi[d]) : 0;
                if (!(j == i && S[0] == 0 && S[1] == 0 && S[2] == 0)) {
                    double v[3];
                    const double r2 = pair_d2(pos, g, i, j, S, v);
                    pass = r2 < rc2_max;
                    in_r = r2 < rc2_r;
                    in_a = r2 < rc2_a;
                    if (pass && !shift_fits(S)) {
                        atomicOr(error_flag, 2);
                        pass = false;
                    }
                }
            }
            const uint64_t bp = __ballot(pass);
            if (pass) {
                const int slot = cu + __popcll(bp & below);
                const uint64_t key = make_key((in_r && in_a) ? 0 : 1, j, S);
                if (slot < cap) out[slot] = key;
                if (slot < KW) kl[wave][slot] = key;
            }
            cu += __popcll(bp);
            cr += __popcll(__ballot(pass && in_r));
            ca += __popcll(__ballot(pass && in_a));
        }
        wave_fence();
    }
    finish_centre<KW>(i, lane, cu, cr, ca, max_r, max_a, cap, kl[wave], out, cnt_union, cnt_r, cnt_a,
                  error_flag);
}

// Re-test of cached candidates at the current positions (the skin reuse of
// rune_nlist_update): one centre per wave, its candidate keys (any class)
// taken 64 at a time with the same exact fp64 test and key packing as
// enumerate_flat, so the centre's row of `keys` comes out identical to a
// fresh enumeration whenever the candidates include every member.
template <int KW>
__global__ void __launch_bounds__(256) refilter_wave(
    int n, const double *pos, const int32_t *sptr, int nstruct, const Geo *geo,
    const uint64_t *cand, int capc, const int32_t *cand_cnt, double rc2_r, double rc2_a,
    double rc2_max, int max_r, int max_a, int cap, int32_t *cnt_union, int32_t *cnt_r,
    int32_t *cnt_a, int32_t *error_flag, uint64_t *keys) {
    __shared__ uint64_t kl[4][KW];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + wave;
    if (i >= n) return;
    const Geo &g = geo[find_structure(sptr, nstruct, i)];
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint64_t *row = cand + size_t(i) * capc;
    uint64_t *out = keys + size_t(i) * cap;
    const int m = cand_cnt[i];
    int cu = 0, cr = 0, ca = 0;
    for (int t0 = 0; t0 < m; t0 += kWave) {
        const int t = t0 + lane;
        bool pass = false, in_r = false, in_a = false;
        int j = 0, S[3] = {0, 0, 0};
        if (t < m) {
            const uint64_t key = row[t];
            j = key_neighbor(key);
            key_shift(key, S);
            double v[3];
            const double r2 = pair_d2(pos, g, i, j, S, v);
            pass = r2 < rc2_max;
            in_r = r2 < rc2_r;
            in_a = r2 < rc2_a;
        }
        const uint64_t bp = __ballot(pass);
        if (pass) {
            const int slot = cu + __popcll(bp & below);
            const uint64_t key = make_key((in_r && in_a) ? 0 : 1, j, S);
            if (slot < cap) out[slot] = key;
            if (slot < KW) kl[wave][slot] = key;
        }
        cu += __popcll(bp);
        cr += __popcll(__ballot(pass && in_r));
        ca += __popcll(__ballot(pass && in_a));
    }
    wave_fence();
    finish_centre<KW>(i, lane, cu, cr, ca, max_r, max_a, cap, kl[wave], out, cnt_union, cnt_r, cnt_a,
                  error_flag);
}

// Sets *flag when some atom moved by skin / 2 or more since the candidate
// search (positions compared as given, so a wrapped atom also triggers it).
__global__ void check_displacement(int n, const double *pos, const double *ref, double limit2,
                                   int32_t *flag) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const double x = pos[3 * i] - ref[3 * i], y = pos[3 * i + 1] - ref[3 * i + 1],
                 z = pos[3 * i + 2] - ref[3 * i + 2];
    if ((x * x + y * y) + z * z >= limit2) atomicOr(flag, 1);
}

// Records of centre i from its sorted keys (row i of keys, stride cap), one
// atom per wave, lanes over its records.
__global__ void __launch_bounds__(256) decode_wave(int n, const double *pos, const int32_t *sptr,
                                                   int nstruct, const Geo *geo, int cap,
                                                   const int32_t *ptr, const int32_t *cnt_r,
                                                   const int32_t *cnt_a, const uint64_t *keys,
                                                   int32_t *view, int32_t *nbr, int32_t *shift,
                                                   float4 *vec, int32_t *ctr, int32_t *indeg) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + wave;
    if (i >= n) return;
    const int s = find_structure(sptr, nstruct, i);
    const Geo &g = geo[s];
    const int b = ptr[i], e = ptr[i + 1];
    if (lane == 0) {
        view[4 * i + 0] = b;
        view[4 * i + 1] = b + cnt_r[i];
        view[4 * i + 2] = b;
        view[4 * i + 3] = b + cnt_a[i];
    }
    const float pi[3] = {float(pos[3 * i]), float(pos[3 * i + 1]), float(pos[3 * i + 2])};
    const uint64_t *row = keys + size_t(i) * cap;
    for (int k = lane; k < e - b; k += kWave) {
        const int r = b + k;
        const uint64_t key = row[k];
        const int j = key_neighbor(key);
        int S[3];
        key_shift(key, S);
        float v[3];
        for (int d = 0; d < 3; ++d) {
            const double o = (double(S[0]) * g.cell[0 * 3 + d] + double(S[1]) * g.cell[1 * 3 + d]) +
                             double(S[2]) * g.cell[2 * 3 + d];
            const float pj = float(pos[3 * j + d]);
            v[d] = (pj + float(o)) - pi[d];
        }
        nbr[r] = j;
        ctr[r] = i;
        atomicAdd(indeg + j, 1);   // in-degree of the transpose
        shift[3 * r + 0] = S[0];
        shift[3 * r + 1] = S[1];
        shift[3 * r + 2] = S[2];
        const float d2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
        vec[r] = make_float4(v[0], v[1], v[2], sqrtf(d2));
    }
}


// ---- records from padded reference batches ----

__global__ void count_padded(int n, const int64_t *rn, int kr, const int64_t *an, int ka,
                             int32_t *cnt_union, int32_t *cnt_r, int32_t *cnt_a) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int cr = 0, ca = 0;
    for (int k = 0; k < kr; ++k) cr += rn[int64_t(i) * kr + k] != -1;
    for (int k = 0; k < ka; ++k) ca += an[int64_t(i) * ka + k] != -1;
    cnt_r[i] = cr;
    cnt_a[i] = ca;
    cnt_union[i] = cr + ca;
}

__global__ void fill_padded(int n, const float *pos, const int64_t *rn, const float *ro, int kr,
                            const int64_t *an, const float *ao, int ka, const int32_t *ptr,
                            const int32_t *cnt_r, const int32_t *cnt_a, int32_t *view,
                            int32_t *nbr, int32_t *shift, float4 *vec, int32_t *ctr) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int b = ptr[i];
    view[4 * i + 0] = b;
    view[4 * i + 1] = b + cnt_r[i];
    view[4 * i + 2] = b + cnt_r[i];
    view[4 * i + 3] = b + cnt_r[i] + cnt_a[i];
    int r = b;
    for (int pass = 0; pass < 2; ++pass) {
        const int64_t *nn = pass ? an : rn;
        const float *oo = pass ? ao : ro;
        int kk = pass ? ka : kr;
        for (int k = 0; k < kk; ++k) {
            int64_t j = nn[int64_t(i) * kk + k];
            if (j == -1) continue;
            const float *o = oo + (int64_t(i) * kk + k) * 3;
            float v[3];
            for (int d = 0; d < 3; ++d) v[d] = (pos[3 * j + d] + o[d]) - pos[3 * i + d];
            nbr[r] = int(j);
            ctr[r] = i;
            shift[3 * r] = shift[3 * r + 1] = shift[3 * r + 2] = 0;
            vec[r] = make_float4(v[0], v[1], v[2], sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]));
            ++r;
        }
    }
}

__global__ void check_padded(int n, int64_t total, const int64_t *rn, int kr, const int64_t *an,
                             int ka, int32_t *error_flag) {
    int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    int64_t v = t < int64_t(n) * kr ? rn[t] : an[t - int64_t(n) * kr];
    if (v < -1 || v >= n) atomicOr(error_flag, 2);
}

// ---- transpose: records grouped by neighbour, ascending record id ----

__global__ void count_in(int64_t e, const int32_t *nbr, int32_t *indeg) {
    int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r < e) atomicAdd(indeg + nbr[r], 1);
}

__global__ void fill_in(int64_t e, const int32_t *nbr, const int32_t *tptr, int32_t *cursor,
                        int32_t *tidx) {
    int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= e) return;
    int a = nbr[r];
    int slot = atomicAdd(cursor + a, 1);
    tidx[tptr[a] + slot] = int(r);
}

// Each atom's transposed records in ascending record order, and the centre
// of each (tctr[t] = ctr[tidx[t]]): one atom per wave, ranked in LDS (record
// ids are distinct, so each value's rank is the number of smaller ones); an
// atom with more than KW falls back to lane 0's insertion sort in global
// memory.
template <int KW>
__global__ void __launch_bounds__(256) sort_in(int n, const int32_t *tptr, int32_t *tidx,
                                               const int32_t *ctr, int32_t *tctr) {
    __shared__ int32_t kl[4][KW];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int a = blockIdx.x * 4 + wave;
    if (a >= n) return;
    int32_t *k = tidx + tptr[a];
    int32_t *kc = tctr + tptr[a];
    const int c = tptr[a + 1] - tptr[a];
    if (c <= KW) {
        for (int p = lane; p < c; p += kWave) kl[wave][p] = k[p];
        wave_fence();
        for (int p = lane; p < c; p += kWave) {
            const int32_t x = kl[wave][p];
            int rank = 0;
            for (int b = 0; b < c; ++b) rank += kl[wave][b] < x ? 1 : 0;
            k[rank] = x;
            kc[rank] = ctr[x];
        }
        return;
    }
    if (lane != 0) return;
    for (int p = 1; p < c; ++p) {
        int32_t x = k[p];
        int q = p - 1;
        while (q >= 0 && k[q] > x) {
            k[q + 1] = k[q];
            --q;
        }
        k[q + 1] = x;
    }
    for (int p = 0; p < c; ++p) kc[p] = ctr[k[p]];
}

// The record total ptr[n] and the builder's flag word, stored straight into
// pinned host memory (read after one stream synchronisation).
__global__ void publish_counts(const int32_t *total, const int32_t *flag, int32_t *host) {
    if (threadIdx.x == 0) {
        host[0] = *total;
        host[1] = *flag;
    }
}

// ---- host helpers ----

void invert3(const double *c, double *inv) {
    double det = c[0] * (c[4] * c[8] - c[5] * c[7]) - c[1] * (c[3] * c[8] - c[5] * c[6]) +
                 c[2] * (c[3] * c[7] - c[4] * c[6]);
    RUNE_REQUIRE(std::fabs(det) > 1e-12, RUNE_ERR_ARGUMENT, "cell is singular");
    double id = 1.0 / det;
    inv[0] = (c[4] * c[8] - c[5] * c[7]) * id;
    inv[1] = (c[2] * c[7] - c[1] * c[8]) * id;
    inv[2] = (c[1] * c[5] - c[2] * c[4]) * id;
    inv[3] = (c[5] * c[6] - c[3] * c[8]) * id;
    inv[4] = (c[0] * c[8] - c[2] * c[6]) * id;
    inv[5] = (c[2] * c[3] - c[0] * c[5]) * id;
    inv[6] = (c[3] * c[7] - c[4] * c[6]) * id;
    inv[7] = (c[1] * c[6] - c[0] * c[7]) * id;
    inv[8] = (c[0] * c[4] - c[1] * c[3]) * id;
}

void cross(const double *a, const double *b, double *o) {
    o[0] = a[1] * b[2] - a[2] * b[1];
    o[1] = a[2] * b[0] - a[0] * b[2];
    o[2] = a[0] * b[1] - a[1] * b[0];
}

double norm3(const double *a) { return std::sqrt(a[0] * a[0] + a[1] * a[1] + a[2] * a[2]); }

// Spreads the low 10 bits of v to every third bit.
static uint32_t spread3(uint32_t v) {
    v &= 0x3ff;
    v = (v | (v << 16)) & 0x030000ff;
    v = (v | (v << 8)) & 0x0300f00f;
    v = (v | (v << 4)) & 0x030c30c3;
    v = (v | (v << 2)) & 0x09249249;
    return v;
}

// Flat bin ids of one structure in Morton (Z-curve) order of their cell
// coordinates: consecutive ranks are spatially compact at every scale.
static void morton_bins(const int nb[3], int bin_offset, std::vector<int32_t> &out) {
    std::vector<std::pair<uint32_t, int32_t>> keys;
    keys.reserve(size_t(nb[0]) * nb[1] * nb[2]);
    for (int a = 0; a < nb[0]; ++a)
        for (int b = 0; b < nb[1]; ++b)
            for (int c = 0; c < nb[2]; ++c)
                keys.push_back({spread3(a) | (spread3(b) << 1) | (spread3(c) << 2),
                                bin_offset + (a * nb[1] + b) * nb[2] + c});
    std::sort(keys.begin(), keys.end());
    for (const auto &k : keys) out.push_back(k.second);
}

// Geometry of one structure: lattice, inverse, thickness and the initial bins
// of width >= rc per direction.  The bin frame is completed by fit_bins.
Geo make_geo(const double *cell_in, const int32_t *pbc, double rc, double *th) {
    Geo g{};
    std::memcpy(g.cell, cell_in, sizeof(g.cell));
    for (int d = 0; d < 3; ++d) g.pbc[d] = pbc[d] ? 1 : 0;
    // a degenerate row in a non-periodic direction gets an orthogonal stand-in:
    // its shift is always 0, so it only sets the scale of the bins there
    for (int d = 0; d < 3; ++d) {
        if (norm3(g.cell + 3 * d) == 0.0) {
            RUNE_REQUIRE(!g.pbc[d], RUNE_ERR_ARGUMENT,
                         "a periodic direction has a zero-length cell vector");
            const double *a = g.cell + 3 * ((d + 1) % 3);
            const double *b = g.cell + 3 * ((d + 2) % 3);
            double c[3];
            cross(a, b, c);
            double nc = norm3(c);
            if (nc == 0.0) {
                for (int k = 0; k < 3; ++k) g.cell[3 * d + k] = (k == d) ? 3.0 * rc : 0.0;
            } else {
                for (int k = 0; k < 3; ++k) g.cell[3 * d + k] = c[k] / nc * 3.0 * rc;
            }
        }
    }
    invert3(g.cell, g.inv);
    double vol = std::fabs(g.cell[0] * (g.cell[4] * g.cell[8] - g.cell[5] * g.cell[7]) -
                           g.cell[1] * (g.cell[3] * g.cell[8] - g.cell[5] * g.cell[6]) +
                           g.cell[2] * (g.cell[3] * g.cell[7] - g.cell[4] * g.cell[6]));
    for (int d = 0; d < 3; ++d) {
        double c[3];
        cross(g.cell + 3 * ((d + 1) % 3), g.cell + 3 * ((d + 2) % 3), c);
        th[d] = vol / norm3(c);
        double nb = std::floor(th[d] / (rc * (1.0 + 1e-9)));
        g.nb[d] = int(std::max(1.0, std::min(nb, 1024.0)));
        g.bs[d] = double(g.nb[d]);
        g.lo[d] = 0.0;
        g.nbin[d] = g.nb[d];
    }
    return g;
}

constexpr double kDenseBin = 12.0;

// Bin frame of one structure.  Periodic directions tile the cell with nb
// bins; open directions cover exactly the bins that hold atoms, from the
// extent [flo, fhi] of the atoms' fractional coordinates (an atom outside
// the cell is never clamped into an edge bin, and a cell-less cluster is
// binned over its own bounding box).  The bin count is capped at 4 per atom
// by halving the finest direction, then the stencil reach follows from the
// bin width th / bs >= rc.
void fit_bins(Geo &g, const double *th, double rc, int n_atoms, const double *flo,
              const double *fhi, int bin_offset, int atom_begin) {
    const int64_t cap = std::max<int64_t>(64, 4 * int64_t(n_atoms));
    // dense periodic cells (on average kDenseBin atoms or more per bin of the
    // cutoff's width) take bins of half that width: the 5x5x5 stencil then
    // proposes about 1.7x fewer candidates than the 3x3x3 one
    if (g.pbc[0] && g.pbc[1] && g.pbc[2] &&
        double(n_atoms) >= kDenseBin * double(g.nb[0]) * double(g.nb[1]) * double(g.nb[2])) {
        for (int d = 0; d < 3; ++d) {
            const double nb = std::floor(2.0 * th[d] / (rc * (1.0 + 1e-9)));
            g.nb[d] = int(std::max(1.0, std::min(nb, 1024.0)));
        }
    }
    for (;;) {
        double total = 1.0;
        for (int d = 0; d < 3; ++d) {
            if (g.pbc[d]) {
                g.bs[d] = double(g.nb[d]);
                g.lo[d] = 0.0;
                g.nbin[d] = g.nb[d];
            } else if (n_atoms > 0) {
                // the same products and floors as the binning kernel
                g.lo[d] = std::floor(flo[d] * g.bs[d]);
                const double span = std::floor(fhi[d] * g.bs[d]) - g.lo[d] + 1.0;
                g.nbin[d] = int(std::min(span, double(int64_t(1) << 30)));
            } else {
                g.lo[d] = 0.0;
                g.nbin[d] = 1;
            }
            total *= double(g.nbin[d]);
        }
        if (total <= double(cap)) break;
        int d = 0;
        for (int k = 1; k < 3; ++k)
            if (g.nbin[k] > g.nbin[d]) d = k;
        if (g.pbc[d])
            g.nb[d] = std::max(1, g.nb[d] / 2);
        else
            g.bs[d] *= 0.5;
    }
    for (int d = 0; d < 3; ++d) {
        g.m[d] = int(std::floor(rc * g.bs[d] / th[d])) + 1;
        if (!g.pbc[d]) g.m[d] = std::min(g.m[d], g.nbin[d]);
        RUNE_REQUIRE(g.m[d] <= 60, RUNE_ERR_ARGUMENT,
                     "cell is too thin for the cutoff (more than 60 images per direction)");
    }
    g.bin_offset = bin_offset;
    g.atom_begin = atom_begin;
    g.atom_end = atom_begin + n_atoms;
}

const char *const kShiftMessage =
    "an atom lies more than 511 cell periods from the cell (periodic image shift outside "
    "[-512, 511]); wrap the positions into the cell";

static double from_ordered_bits(uint64_t k) {
    const uint64_t u = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
    double x;
    std::memcpy(&x, &u, sizeof(x));
    return x;
}

// Upload of a small host array to `dev`, skipped when the device copy
// already holds these bytes (`shadow` keeps what was last uploaded; a
// reallocation of `dev` forces the upload).  Repeated builds of one system
// then issue no host-to-device copies.
void upload_cached(rune::DeviceBuffer &dev, std::vector<char> &shadow, const void *src,
                   size_t bytes, hipStream_t s) {
    void *before = dev.ptr;
    dev.reserve(std::max<size_t>(bytes, 1));
    if (dev.ptr == before && shadow.size() == bytes &&
        (bytes == 0 || std::memcmp(shadow.data(), src, bytes) == 0))
        return;
    shadow.assign(static_cast<const char *>(src), static_cast<const char *>(src) + bytes);
    if (bytes)
        RUNE_HIP_CHECK(hipMemcpyAsync(dev.ptr, shadow.data(), bytes, hipMemcpyHostToDevice, s));
}

// Atom count from which the builder computes the Morton processing order.
constexpr int kOrderMinAtoms = 4096;

struct Work {
    int32_t *atom_bin, *atom_wrap, *atom_cell, *bin_count, *bin_start, *bin_cursor, *bin_atoms;
    int32_t *cnt_union, *cnt_r, *cnt_a, *flag, *scan_tmp, *indeg;
    Geo *geo;
};

// indeg and cursor: n + 1 counters each, cleared by the caller (inside its
// one clearing of the builder's counters); `counted`: indeg already holds
// the in-degrees (counted while the records were written); `cap`: the
// largest in-degree expected (larger ones take a slower sort, still exact).
void build_transpose(rune_nlist *nl, int32_t *indeg, int32_t *cursor, int32_t *scan_tmp,
                     bool counted, int cap, hipStream_t s) {
    int n = int(nl->n_atoms);
    int64_t e = nl->n_records;
    nl->tptr.reserve(sizeof(int32_t) * (n + 1));
    nl->tidx.reserve(sizeof(int32_t) * std::max<int64_t>(e, 1));
    if (e > 0 && !counted)
        hipLaunchKernelGGL(count_in, dim3(ceil_div(e, kThreads)), dim3(kThreads), 0, s, e,
                           nl->nbr.as<int32_t>(), indeg);
    exclusive_scan(indeg, nl->tptr.as<int32_t>(), n, scan_tmp, s);
    if (e > 0) {
        hipLaunchKernelGGL(fill_in, dim3(ceil_div(e, kThreads)), dim3(kThreads), 0, s, e,
                           nl->nbr.as<int32_t>(), nl->tptr.as<int32_t>(), cursor,
                           nl->tidx.as<int32_t>());
        nl->tctr.reserve(sizeof(int32_t) * std::max<int64_t>(e, 1));
        by_key_lds(cap, [&](auto kw) {
            hipLaunchKernelGGL(sort_in<decltype(kw)::value>, dim3(ceil_div(n, 4)), dim3(256), 0,
                               s, n, nl->tptr.as<int32_t>(), nl->tidx.as<int32_t>(),
                               nl->ctr.as<int32_t>(), nl->tctr.as<int32_t>());
        });
    } else {
        nl->tctr.reserve(sizeof(int32_t));
    }
    RUNE_HIP_CHECK(hipGetLastError());
}

std::string overflow_message(const std::vector<int32_t> &cr, const std::vector<int32_t> &ca,
                             int max_r, int max_a) {
    // the reference checks the radial list first (batch.py:83-96, :20-33)
    for (int pass = 0; pass < 2; ++pass) {
        const std::vector<int32_t> &c = pass ? ca : cr;
        int cap = pass ? max_a : max_r;
        int best = 0, atom = 0;
        for (size_t i = 0; i < c.size(); ++i)
            if (c[i] > best) {
                best = c[i];
                atom = int(i);
            }
        if (best > cap) {
            std::ostringstream os;
            os << "Neighbor count " << best << " for atom " << atom
               << " exceeds max_neighbors=" << cap
               << ". Increase max_neighbors_radial or max_neighbors_angular.";
            return os.str();
        }
    }
    return "neighbour capacity exceeded";
}

}  // namespace
}  // namespace rune

using namespace rune;

extern "C" int rune_nlist_create(rune_nlist **out) {
    return guarded([&] {
        RUNE_REQUIRE(out, RUNE_ERR_ARGUMENT, "null output pointer");
        *out = new rune_nlist();
    });
}

extern "C" void rune_nlist_destroy(rune_nlist *nl) { delete nl; }

extern "C" int64_t rune_nlist_atoms(const rune_nlist *nl) { return nl ? nl->n_atoms : 0; }
extern "C" int64_t rune_nlist_records(const rune_nlist *nl) { return nl ? nl->n_records : 0; }

static void set_structures(rune_nlist *nl, int64_t n_atoms, int32_t nstruct,
                           const int64_t *h_sptr, hipStream_t s) {
    RUNE_REQUIRE(nstruct >= 1 && h_sptr, RUNE_ERR_ARGUMENT, "need at least one structure");
    RUNE_REQUIRE(h_sptr[0] == 0 && h_sptr[nstruct] == n_atoms, RUNE_ERR_ARGUMENT,
                 "structure ranges must cover all atoms");
    for (int b = 0; b < nstruct; ++b)
        RUNE_REQUIRE(h_sptr[b + 1] >= h_sptr[b], RUNE_ERR_ARGUMENT,
                     "structure ranges must be non-decreasing");
    RUNE_REQUIRE(n_atoms < (int64_t(1) << 30), RUNE_ERR_ARGUMENT, "too many atoms");
    nl->h_struct_ptr.assign(h_sptr, h_sptr + nstruct + 1);
    std::vector<int32_t> sp(nstruct + 1);
    for (int b = 0; b <= nstruct; ++b) sp[b] = int32_t(h_sptr[b]);
    upload_cached(nl->sptr, nl->sptr_shadow, sp.data(), sizeof(int32_t) * (nstruct + 1), s);
    nl->n_structures = nstruct;
    nl->n_atoms = n_atoms;
}

// Shared body of rune_nlist_build and rune_nlist_update.  skin == 0: one
// enumeration at the model cutoffs.  skin > 0: when `search` is set, the
// candidates within max(rc) + skin are enumerated into nl->cand_keys (and the
// positions kept in nl->ref_pos); either way the candidates are then re-tested
// at the current positions into nl->keys.  The rest (counts, records,
// transpose) is the same for all paths, so all give identical records.
static void build_lists(rune_nlist *nl, int64_t n_atoms, const double *d_positions,
                        int32_t n_structures, const int64_t *h_struct_ptr, const double *h_cells,
                        const int32_t *h_pbc, double rc_radial, double rc_angular,
                        int32_t max_radial, int32_t max_angular, double skin, bool search,
                        hipStream_t s, int64_t *n_records) {
    set_structures(nl, n_atoms, n_structures, h_struct_ptr, s);
    nl->rc_radial = rc_radial;
    nl->rc_angular = rc_angular;
    nl->from_padded = false;
    const int n = int(n_atoms);
    const double rc = std::max(rc_radial, rc_angular), rc_bin = rc + skin;
    std::vector<Geo> geo(n_structures);
    std::vector<double> th(3 * size_t(n_structures));
    bool open = false;
    for (int b = 0; b < n_structures; ++b) {
        geo[b] = make_geo(h_cells + 9 * b, h_pbc + 3 * b, rc_bin, th.data() + 3 * b);
        const bool has_atoms = h_struct_ptr[b + 1] > h_struct_ptr[b];
        open = open || (has_atoms && !(geo[b].pbc[0] && geo[b].pbc[1] && geo[b].pbc[2]));
    }
    // extent of the atoms along open directions (one readback, only when a
    // structure with atoms has a non-periodic direction)
    const bool binned = skin == 0.0 || search;
    std::vector<double> ext(6 * size_t(n_structures), 0.0);
    if (open && binned && n > 0) {
        nl->extent.reserve(sizeof(Geo) * n_structures + 48 * size_t(n_structures));
        Geo *d_geo = nl->extent.as<Geo>();
        auto *d_ext = reinterpret_cast<unsigned long long *>(
            nl->extent.as<char>() + sizeof(Geo) * n_structures);
        RUNE_HIP_CHECK(hipMemcpyAsync(d_geo, geo.data(), sizeof(Geo) * n_structures,
                                      hipMemcpyHostToDevice, s));
        RUNE_HIP_CHECK(hipMemsetAsync(d_ext, 0xff, 24 * size_t(n_structures), s));
        RUNE_HIP_CHECK(hipMemsetAsync(d_ext + 3 * n_structures, 0x00, 24 * size_t(n_structures),
                                      s));
        hipLaunchKernelGGL(frac_extent, dim3(ceil_div(n, kThreads)), dim3(kThreads), 0, s, n,
                           d_positions, nl->sptr.as<int32_t>(), n_structures, d_geo, d_ext);
        RUNE_HIP_CHECK(hipGetLastError());
        std::vector<uint64_t> bits(6 * size_t(n_structures));
        RUNE_HIP_CHECK(hipMemcpyAsync(bits.data(), d_ext, 48 * size_t(n_structures),
                                      hipMemcpyDeviceToHost, s));
        RUNE_HIP_CHECK(hipStreamSynchronize(s));
        for (int b = 0; b < n_structures; ++b)
            for (int d = 0; d < 3; ++d) {
                const bool has_atoms = h_struct_ptr[b + 1] > h_struct_ptr[b];
                const double lo = from_ordered_bits(bits[3 * b + d]);
                const double hi = from_ordered_bits(bits[3 * (n_structures + b) + d]);
                RUNE_REQUIRE(geo[b].pbc[d] || !has_atoms || (std::isfinite(lo) && std::isfinite(hi)),
                             RUNE_ERR_ARGUMENT, "atom positions must be finite");
                ext[6 * b + d] = lo;
                ext[6 * b + 3 + d] = hi;
            }
    }
    int total_bins = 0;
    for (int b = 0; b < n_structures; ++b) {
        int na = int(h_struct_ptr[b + 1] - h_struct_ptr[b]);
        fit_bins(geo[b], th.data() + 3 * b, rc_bin, na, ext.data() + 6 * b,
                 ext.data() + 6 * b + 3, total_bins, int(h_struct_ptr[b]));
        total_bins += geo[b].nbin[0] * geo[b].nbin[1] * geo[b].nbin[2];
    }
    // working memory
    // (the counters that start at zero come first, so one fill clears them)
    Arena ar;
    size_t o_flag = ar.add(16);
    size_t o_bcnt = ar.add(4 * size_t(total_bins + 1));
    size_t o_bcur = ar.add(4 * size_t(total_bins + 1));
    size_t o_indeg = ar.add(4 * size_t(n + 1));
    size_t o_tcur = ar.add(4 * size_t(n + 1));
    const size_t zero_bytes = ar.total;
    size_t o_abin = ar.add(4 * size_t(n + 1));
    size_t o_wrap = ar.add(12 * size_t(n + 1));
    size_t o_cell = ar.add(12 * size_t(n + 1));
    size_t o_bst = ar.add(4 * size_t(total_bins + 2));
    size_t o_batm = ar.add(4 * size_t(n + 1));
    size_t o_cu = ar.add(4 * size_t(n + 1));
    size_t o_cr = ar.add(4 * size_t(n + 1));
    size_t o_ca = ar.add(4 * size_t(n + 1));
    size_t o_scan = ar.add(4 * scan_tmp_ints(std::max(n, total_bins) + 1));
    size_t o_rcnt = ar.add(4 * size_t(total_bins + 1));
    size_t o_rst = ar.add(4 * size_t(total_bins + 2));
    nl->work.reserve(ar.total);
    char *base = nl->work.as<char>();
    Work w;
    upload_cached(nl->geo, nl->geo_shadow, geo.data(), sizeof(Geo) * n_structures, s);
    w.geo = nl->geo.as<Geo>();
    w.atom_bin = reinterpret_cast<int32_t *>(base + o_abin);
    w.atom_wrap = reinterpret_cast<int32_t *>(base + o_wrap);
    w.atom_cell = reinterpret_cast<int32_t *>(base + o_cell);
    w.bin_count = reinterpret_cast<int32_t *>(base + o_bcnt);
    w.bin_start = reinterpret_cast<int32_t *>(base + o_bst);
    w.bin_cursor = reinterpret_cast<int32_t *>(base + o_bcur);
    w.bin_atoms = reinterpret_cast<int32_t *>(base + o_batm);
    w.cnt_union = reinterpret_cast<int32_t *>(base + o_cu);
    w.cnt_r = reinterpret_cast<int32_t *>(base + o_cr);
    w.cnt_a = reinterpret_cast<int32_t *>(base + o_ca);
    w.flag = reinterpret_cast<int32_t *>(base + o_flag);
    w.scan_tmp = reinterpret_cast<int32_t *>(base + o_scan);
    w.indeg = reinterpret_cast<int32_t *>(base + o_indeg);
    int32_t *tcur = reinterpret_cast<int32_t *>(base + o_tcur);
    RUNE_HIP_CHECK(hipMemsetAsync(base, 0, zero_bytes, s));
    nl->ptr.reserve(4 * size_t(n + 1));
    nl->view.reserve(16 * size_t(n + 1));
    int gb = ceil_div(std::max(n, 1), kThreads);
    const int32_t *sptr = nl->sptr.as<int32_t>();
    // one row of sorted keys per centre, as wide as the larger neighbour limit
    const int cap = std::max(max_radial, max_angular);
    nl->keys.reserve(8 * size_t(std::max(n, 1)) * size_t(cap));
    const double rc2_r = rc_radial * rc_radial, rc2_a = rc_angular * rc_angular, rc2 = rc * rc;
    if (binned) {
        if (n > 0)
            hipLaunchKernelGGL(bin_atoms, dim3(gb), dim3(kThreads), 0, s, n, d_positions, sptr,
                               n_structures, w.geo, w.atom_bin, w.atom_wrap, w.atom_cell,
                               w.bin_count);
        exclusive_scan(w.bin_count, w.bin_start, total_bins, w.scan_tmp, s);
        if (n > 0)
            hipLaunchKernelGGL(fill_bins, dim3(gb), dim3(kThreads), 0, s, n, w.atom_bin,
                               w.bin_start, w.bin_cursor, w.bin_atoms);
    }
    if (skin == 0.0) {
        if (n > 0)
            by_key_lds(cap, [&](auto kw) {
                hipLaunchKernelGGL(enumerate_flat<decltype(kw)::value>, dim3(ceil_div(n, 4)),
                                   dim3(256), 0, s, n, d_positions, sptr, n_structures, w.geo,
                                   w.atom_wrap, w.atom_cell, w.bin_start, w.bin_atoms, rc2_r,
                                   rc2_a, rc2, max_radial, max_angular, cap, w.cnt_union,
                                   w.cnt_r, w.cnt_a, w.flag, nl->keys.as<uint64_t>());
            });
    } else {
        if (search) {
            // candidates within rc + skin, all of class 0 (sorted by (j, S));
            // a row that overflows the candidate width widens it and repeats
            const double rb2 = rc_bin * rc_bin;
            nl->cand_cnt.reserve(4 * size_t(n + 1));
            for (int attempt = 0;; ++attempt) {
                nl->cand_keys.reserve(8 * size_t(std::max(n, 1)) * size_t(nl->cand_cap));
                if (n > 0)
                    by_key_lds(nl->cand_cap, [&](auto kw) {
                        hipLaunchKernelGGL(enumerate_flat<decltype(kw)::value>,
                                           dim3(ceil_div(n, 4)), dim3(256), 0, s, n, d_positions,
                                           sptr, n_structures, w.geo, w.atom_wrap, w.atom_cell,
                                           w.bin_start, w.bin_atoms, rb2, rb2, rb2, nl->cand_cap,
                                           nl->cand_cap, nl->cand_cap,
                                           nl->cand_cnt.as<int32_t>(), w.cnt_r, w.cnt_a, w.flag,
                                           nl->cand_keys.as<uint64_t>());
                    });
                RUNE_HIP_CHECK(hipGetLastError());
                int32_t over = 0;
                RUNE_HIP_CHECK(hipMemcpyAsync(&over, w.flag, 4, hipMemcpyDeviceToHost, s));
                RUNE_HIP_CHECK(hipStreamSynchronize(s));
                RUNE_REQUIRE(!(over & 2), RUNE_ERR_ARGUMENT, kShiftMessage);
                if (!over) break;
                RUNE_REQUIRE(attempt < 3, RUNE_ERR_STATE, "neighbour candidate search did not fit");
                std::vector<int32_t> cc(n);
                RUNE_HIP_CHECK(hipMemcpy(cc.data(), nl->cand_cnt.ptr, 4 * size_t(n),
                                         hipMemcpyDeviceToHost));
                const int most = n ? *std::max_element(cc.begin(), cc.end()) : 0;
                nl->cand_cap = std::max(nl->cand_cap + 1, most + most / 4 + 8);
                RUNE_HIP_CHECK(hipMemsetAsync(w.flag, 0, 16, s));
            }
            nl->ref_pos.reserve(24 * size_t(std::max(n, 1)));
            if (n > 0)
                RUNE_HIP_CHECK(hipMemcpyAsync(nl->ref_pos.ptr, d_positions, 24 * size_t(n),
                                              hipMemcpyDeviceToDevice, s));
        }
        if (n > 0)
            by_key_lds(cap, [&](auto kw) {
                hipLaunchKernelGGL(refilter_wave<decltype(kw)::value>, dim3(ceil_div(n, 4)),
                                   dim3(256), 0, s, n, d_positions, sptr, n_structures, w.geo,
                                   nl->cand_keys.as<uint64_t>(), nl->cand_cap,
                                   nl->cand_cnt.as<int32_t>(), rc2_r, rc2_a, rc2, max_radial,
                                   max_angular, cap, w.cnt_union, w.cnt_r, w.cnt_a, w.flag,
                                   nl->keys.as<uint64_t>());
            });
    }
    exclusive_scan(w.cnt_union, nl->ptr.as<int32_t>(), n, w.scan_tmp, s);
    int32_t *words = nl->readback.get();
    hipLaunchKernelGGL(publish_counts, dim3(1), dim3(64), 0, s, nl->ptr.as<int32_t>() + n, w.flag,
                       words);
    RUNE_HIP_CHECK(hipGetLastError());
    RUNE_HIP_CHECK(hipStreamSynchronize(s));
    const int32_t host[2] = {nl->readback.read(0), nl->readback.read(1)};
    RUNE_REQUIRE(!(host[1] & 2), RUNE_ERR_ARGUMENT, kShiftMessage);
    if (host[1]) {
        std::vector<int32_t> cr(n), ca(n);
        RUNE_HIP_CHECK(hipMemcpy(cr.data(), w.cnt_r, 4 * size_t(n), hipMemcpyDeviceToHost));
        RUNE_HIP_CHECK(hipMemcpy(ca.data(), w.cnt_a, 4 * size_t(n), hipMemcpyDeviceToHost));
        nl->n_records = 0;
        throw Error(RUNE_ERR_OVERFLOW, overflow_message(cr, ca, max_radial, max_angular));
    }
    int64_t e = host[0];
    nl->n_records = e;
    size_t ecap = size_t(std::max<int64_t>(e, 1));
    nl->nbr.reserve(4 * ecap);
    nl->shift.reserve(12 * ecap);
    nl->vec.reserve(16 * ecap);
    nl->ctr.reserve(4 * ecap);
    if (n > 0) {
        hipLaunchKernelGGL(decode_wave, dim3(ceil_div(n, 4)), dim3(256), 0, s, n, d_positions,
                           sptr, n_structures, w.geo, cap, nl->ptr.as<int32_t>(), w.cnt_r,
                           w.cnt_a, nl->keys.as<uint64_t>(), nl->view.as<int32_t>(),
                           nl->nbr.as<int32_t>(), nl->shift.as<int32_t>(), nl->vec.as<float4>(),
                           nl->ctr.as<int32_t>(), w.indeg);
    }
    RUNE_HIP_CHECK(hipGetLastError());
    build_transpose(nl, w.indeg, tcur, w.scan_tmp, true, cap, s);
    // processing order: atoms bin by bin, bins in Morton order (kept from the
    // last binning when the candidates are reused; it only orders the work,
    // so a list of fewer than kOrderMinAtoms atoms, which fits in L2 either
    // way, keeps the index order and saves the launches)
    if (binned && (n < kOrderMinAtoms || !nl->order_wanted)) {
        nl->has_order = false;
    } else if (binned) {
        nl->order.reserve(4 * size_t(std::max(n, 1)));
        if (n > 0) {
            // the bin ranks depend only on the bin grids: recomputed and
            // uploaded when those changed
            const size_t gbytes = sizeof(Geo) * n_structures;
            if (nl->perm_geo.size() != gbytes ||
                std::memcmp(nl->perm_geo.data(), geo.data(), gbytes) != 0) {
                nl->h_perm.clear();
                nl->h_perm.reserve(total_bins);
                for (int b = 0; b < n_structures; ++b)
                    morton_bins(geo[b].nbin, geo[b].bin_offset, nl->h_perm);
                nl->perm_geo.assign(reinterpret_cast<const char *>(geo.data()),
                                    reinterpret_cast<const char *>(geo.data()) + gbytes);
            }
            upload_cached(nl->perm, nl->perm_shadow, nl->h_perm.data(),
                          4 * nl->h_perm.size(), s);
            int32_t *d_perm = nl->perm.as<int32_t>();
            int32_t *rcnt = reinterpret_cast<int32_t *>(base + o_rcnt);
            int32_t *rst = reinterpret_cast<int32_t *>(base + o_rst);
            const int bg = ceil_div(total_bins, kThreads);
            hipLaunchKernelGGL(rank_counts, dim3(bg), dim3(kThreads), 0, s, total_bins, d_perm,
                               w.bin_count, rcnt);
            exclusive_scan(rcnt, rst, total_bins, w.scan_tmp, s);
            hipLaunchKernelGGL(order_atoms, dim3(bg), dim3(kThreads), 0, s, total_bins, d_perm,
                               w.bin_start, w.bin_count, rst, w.bin_atoms,
                               nl->order.as<int32_t>());
            RUNE_HIP_CHECK(hipGetLastError());
        }
        nl->has_order = true;
    }
    if (n_records) *n_records = e;
}

static void check_build_args(rune_nlist *nl, int64_t n_atoms, const double *d_positions,
                             const double *h_cells, const int32_t *h_pbc, double rc_radial,
                             double rc_angular, int32_t max_radial, int32_t max_angular) {
    RUNE_REQUIRE(nl && (d_positions || n_atoms == 0) && h_cells && h_pbc, RUNE_ERR_ARGUMENT,
                 "null argument");
    RUNE_REQUIRE(rc_radial > 0 && rc_angular > 0, RUNE_ERR_ARGUMENT,
                 "radial and angular cutoffs must be positive");
    RUNE_REQUIRE(max_radial >= 1 && max_angular >= 1, RUNE_ERR_ARGUMENT,
                 "radial and angular max-neighbor counts must be positive");
}

extern "C" int rune_nlist_build(rune_nlist *nl, int64_t n_atoms, const double *d_positions,
                                int32_t n_structures, const int64_t *h_struct_ptr,
                                const double *h_cells, const int32_t *h_pbc, double rc_radial,
                                double rc_angular, int32_t max_radial, int32_t max_angular,
                                void *stream, int64_t *n_records) {
    return guarded([&] {
        check_build_args(nl, n_atoms, d_positions, h_cells, h_pbc, rc_radial, rc_angular,
                         max_radial, max_angular);
        nl->cand_valid = false;
        build_lists(nl, n_atoms, d_positions, n_structures, h_struct_ptr, h_cells, h_pbc,
                    rc_radial, rc_angular, max_radial, max_angular, 0.0, true, as_stream(stream),
                    n_records);
    });
}

extern "C" int rune_nlist_update(rune_nlist *nl, int64_t n_atoms, const double *d_positions,
                                 int32_t n_structures, const int64_t *h_struct_ptr,
                                 const double *h_cells, const int32_t *h_pbc, double rc_radial,
                                 double rc_angular, int32_t max_radial, int32_t max_angular,
                                 double skin, void *stream, int64_t *n_records,
                                 int32_t *searched) {
    return guarded([&] {
        check_build_args(nl, n_atoms, d_positions, h_cells, h_pbc, rc_radial, rc_angular,
                         max_radial, max_angular);
        RUNE_REQUIRE(skin > 0 && std::isfinite(skin), RUNE_ERR_ARGUMENT, "skin must be positive");
        RUNE_REQUIRE(n_structures >= 1 && h_struct_ptr, RUNE_ERR_ARGUMENT,
                     "need at least one structure");
        hipStream_t s = as_stream(stream);
        // everything the candidates depend on besides the positions
        std::vector<double> key;
        key.reserve(6 + 13 * size_t(n_structures));
        key.insert(key.end(), {double(n_atoms), rc_radial, rc_angular, double(max_radial),
                               double(max_angular), skin});
        for (int b = 0; b < n_structures; ++b) {
            key.push_back(double(h_struct_ptr[b + 1]));
            key.insert(key.end(), h_cells + 9 * b, h_cells + 9 * b + 9);
            for (int d = 0; d < 3; ++d) key.push_back(h_pbc[3 * b + d] ? 1.0 : 0.0);
        }
        bool search = !nl->cand_valid || key != nl->cand_key;
        if (!search && n_atoms > 0) {
            int32_t *flag = nl->cand_flag.as<int32_t>();
            RUNE_HIP_CHECK(hipMemsetAsync(flag, 0, 4, s));
            hipLaunchKernelGGL(check_displacement, dim3(ceil_div(n_atoms, kThreads)),
                               dim3(kThreads), 0, s, int(n_atoms), d_positions,
                               nl->ref_pos.as<double>(), 0.25 * skin * skin, flag);
            RUNE_HIP_CHECK(hipGetLastError());
            int32_t moved = 0;
            RUNE_HIP_CHECK(hipMemcpyAsync(&moved, flag, 4, hipMemcpyDeviceToHost, s));
            RUNE_HIP_CHECK(hipStreamSynchronize(s));
            search = moved != 0;
        }
        nl->cand_valid = false;
        if (nl->cand_cap < 1) nl->cand_cap = std::max(max_radial, max_angular);
        nl->cand_flag.reserve(16);
        build_lists(nl, n_atoms, d_positions, n_structures, h_struct_ptr, h_cells, h_pbc,
                    rc_radial, rc_angular, max_radial, max_angular, skin, search, s, n_records);
        nl->cand_key = key;
        nl->cand_valid = true;
        if (searched) *searched = search ? 1 : 0;
    });
}

extern "C" int rune_nlist_from_padded(rune_nlist *nl, int64_t n_atoms, const float *d_positions,
                                      const int64_t *d_radial_nbr, const float *d_radial_off,
                                      int32_t k_radial, const int64_t *d_angular_nbr,
                                      const float *d_angular_off, int32_t k_angular,
                                      int32_t n_structures, const int64_t *h_struct_ptr,
                                      void *stream, int64_t *n_records) {
    return guarded([&] {
        RUNE_REQUIRE(nl, RUNE_ERR_ARGUMENT, "null handle");
        RUNE_REQUIRE(k_radial >= 0 && k_angular >= 0, RUNE_ERR_ARGUMENT, "negative width");
        hipStream_t s = as_stream(stream);
        set_structures(nl, n_atoms, n_structures, h_struct_ptr, s);
        nl->from_padded = true;
        nl->has_order = false;
        const int n = int(n_atoms);
        Arena ar;
        size_t o_flag = ar.add(16);
        size_t o_indeg = ar.add(4 * size_t(n + 1));
        size_t o_tcur = ar.add(4 * size_t(n + 1));
        const size_t zero_bytes = ar.total;
        size_t o_cu = ar.add(4 * size_t(n + 1));
        size_t o_cr = ar.add(4 * size_t(n + 1));
        size_t o_ca = ar.add(4 * size_t(n + 1));
        size_t o_scan = ar.add(4 * scan_tmp_ints(n + 1));
        nl->work.reserve(ar.total);
        char *base = nl->work.as<char>();
        int32_t *cu = reinterpret_cast<int32_t *>(base + o_cu);
        int32_t *cr = reinterpret_cast<int32_t *>(base + o_cr);
        int32_t *ca = reinterpret_cast<int32_t *>(base + o_ca);
        int32_t *flag = reinterpret_cast<int32_t *>(base + o_flag);
        int32_t *scan_tmp = reinterpret_cast<int32_t *>(base + o_scan);
        int32_t *indeg = reinterpret_cast<int32_t *>(base + o_indeg);
        int32_t *tcur = reinterpret_cast<int32_t *>(base + o_tcur);
        RUNE_HIP_CHECK(hipMemsetAsync(base, 0, zero_bytes, s));
        nl->ptr.reserve(4 * size_t(n + 1));
        nl->view.reserve(16 * size_t(n + 1));
        int gb = ceil_div(std::max(n, 1), kThreads);
        int64_t slots = int64_t(n) * (k_radial + k_angular);
        if (slots > 0)
            hipLaunchKernelGGL(check_padded, dim3(ceil_div(slots, kThreads)), dim3(kThreads), 0,
                               s, n, slots, d_radial_nbr, k_radial, d_angular_nbr, k_angular,
                               flag);
        if (n > 0)
            hipLaunchKernelGGL(count_padded, dim3(gb), dim3(kThreads), 0, s, n, d_radial_nbr,
                               k_radial, d_angular_nbr, k_angular, cu, cr, ca);
        exclusive_scan(cu, nl->ptr.as<int32_t>(), n, scan_tmp, s);
        int32_t host[2] = {0, 0};
        RUNE_HIP_CHECK(hipMemcpyAsync(&host[0], nl->ptr.as<int32_t>() + n, 4,
                                      hipMemcpyDeviceToHost, s));
        RUNE_HIP_CHECK(hipMemcpyAsync(&host[1], flag, 4, hipMemcpyDeviceToHost, s));
        RUNE_HIP_CHECK(hipStreamSynchronize(s));
        RUNE_REQUIRE(host[1] == 0, RUNE_ERR_ARGUMENT,
                     "neighbour index out of range in padded neighbour list");
        int64_t e = host[0];
        nl->n_records = e;
        size_t ecap = size_t(std::max<int64_t>(e, 1));
        nl->nbr.reserve(4 * ecap);
        nl->shift.reserve(12 * ecap);
        nl->vec.reserve(16 * ecap);
        nl->ctr.reserve(4 * ecap);
        if (n > 0)
            hipLaunchKernelGGL(fill_padded, dim3(gb), dim3(kThreads), 0, s, n, d_positions,
                               d_radial_nbr, d_radial_off, k_radial, d_angular_nbr,
                               d_angular_off, k_angular, nl->ptr.as<int32_t>(), cr, ca,
                               nl->view.as<int32_t>(), nl->nbr.as<int32_t>(),
                               nl->shift.as<int32_t>(), nl->vec.as<float4>(),
                               nl->ctr.as<int32_t>());
        RUNE_HIP_CHECK(hipGetLastError());
        build_transpose(nl, indeg, tcur, scan_tmp, false, kWaveKeys, s);
        if (n_records) *n_records = e;
    });
}

extern "C" int rune_nlist_export(const rune_nlist *nl, int32_t *d_ptr, int32_t *d_view,
                                 int32_t *d_nbr, int32_t *d_shift, float *d_vec, void *stream) {
    return guarded([&] {
        RUNE_REQUIRE(nl, RUNE_ERR_ARGUMENT, "null handle");
        hipStream_t s = as_stream(stream);
        size_t n = size_t(nl->n_atoms), e = size_t(nl->n_records);
        if (d_ptr)
            RUNE_HIP_CHECK(hipMemcpyAsync(d_ptr, nl->ptr.ptr, 4 * (n + 1),
                                          hipMemcpyDeviceToDevice, s));
        if (d_view && n)
            RUNE_HIP_CHECK(hipMemcpyAsync(d_view, nl->view.ptr, 16 * n, hipMemcpyDeviceToDevice, s));
        if (e) {
            if (d_nbr)
                RUNE_HIP_CHECK(hipMemcpyAsync(d_nbr, nl->nbr.ptr, 4 * e, hipMemcpyDeviceToDevice, s));
            if (d_shift)
                RUNE_HIP_CHECK(hipMemcpyAsync(d_shift, nl->shift.ptr, 12 * e,
                                              hipMemcpyDeviceToDevice, s));
            if (d_vec)
                RUNE_HIP_CHECK(hipMemcpyAsync(d_vec, nl->vec.ptr, 16 * e, hipMemcpyDeviceToDevice, s));
        }
    });
}
