// K7: forces and virials from per-record gradients g = dE/dr_ij, without atomics.
//
// F_i = sum_{e: centre i} g_e - sum_{e: neighbour i} g_e   (force.py:151-162,
// model.py:23-44) using the neighbour-grouped transpose list, and the per-atom
// virial W_a = -sum_{e: neighbour a} g_e (x) r_e attributed to the neighbour
// like the reference.  Structure totals use a fixed-order fp64 reduction.
#include <algorithm>

#include "kernels.hpp"

namespace rune {
namespace {

// Eight lanes per atom: lane j of the atom's group takes records j, j + 8,
// ... of its own list (+g) and of its transposed list (-g, virial), then the
// group sums with a fixed xor tree, so the result is the same on every call.
constexpr int kForceLanes = 8;

__global__ void __launch_bounds__(256) k_forces(Records r, const float4 *g, float *forces,
                                                float *atom_virial) {
    const int tid = blockIdx.x * blockDim.x + threadIdx.x;
    const int i = tid / kForceLanes, j = tid % kForceLanes;
    const bool on = i < r.n_atoms;
    float f[3] = {0.0f, 0.0f, 0.0f};
    float w[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (on) {
        for (int e = r.ptr[i] + j; e < r.ptr[i + 1]; e += kForceLanes) {
            const float4 v = g[e];
            f[0] += v.x;
            f[1] += v.y;
            f[2] += v.z;
        }
        for (int t = r.tptr[i] + j; t < r.tptr[i + 1]; t += kForceLanes) {
            const int e = r.tidx[t];
            const float4 v = g[e];
            f[0] -= v.x;
            f[1] -= v.y;
            f[2] -= v.z;
            if (atom_virial) {
                const float4 d = r.vec[e];
                const float gv[3] = {v.x, v.y, v.z}, rv[3] = {d.x, d.y, d.z};
#pragma unroll
                for (int a = 0; a < 3; ++a)
#pragma unroll
                    for (int b = 0; b < 3; ++b) w[3 * a + b] -= gv[a] * rv[b];
            }
        }
    }
    // every lane of the wave takes part in the shuffles
#pragma unroll
    for (int off = kForceLanes / 2; off > 0; off >>= 1) {
#pragma unroll
        for (int a = 0; a < 3; ++a) f[a] += __shfl_xor(f[a], off, kForceLanes);
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] += __shfl_xor(w[k], off, kForceLanes);
    }
    if (!on || j != 0) return;
    if (forces) {
        forces[3 * i + 0] = f[0];
        forces[3 * i + 1] = f[1];
        forces[3 * i + 2] = f[2];
    }
    if (atom_virial)
        for (int k = 0; k < 9; ++k) atom_virial[9 * size_t(i) + k] = w[k];
}

// One workgroup per structure; thread t sums atoms t, t+256, ... then a tree.
// Column sums of x [atoms, ncol] over the atoms of each structure, in fp64.
// Block (p, b, z) takes part p of structure b's atoms for output z (z = 0:
// energies, one column; z = 1: virials, nine columns) and reads them as one
// flat coalesced range; the threads in use are a multiple of the column
// count, so thread t always meets column t % ncol.  The per-thread partials
// of each column are combined by a fixed tree.  With one part the result
// goes to the output, else to part[z][b, p, :].
__global__ void __launch_bounds__(1024) k_structure_sum(const int32_t *sptr, SumArgs a) {
    __shared__ double lds[1024];
    const int b = blockIdx.y, p = blockIdx.x, t = threadIdx.x, z = blockIdx.z;
    const float *x = z ? a.virial : a.energies;
    float *out = z ? a.d_virial : a.d_energy;
    if (!out) return;   // uniform per block
    const int ncol = z ? 9 : 1, parts = a.parts;
    const int per = 1024 / ncol, lanes = per * ncol;
    const int a0 = sptr[b], n = sptr[b + 1] - a0, chunk = (n + parts - 1) / parts;
    const int lo = a0 + min(n, p * chunk), hi = a0 + min(n, (p + 1) * chunk);
    const int64_t beg = int64_t(lo) * ncol, end = int64_t(hi) * ncol;
    double s = 0.0;
    if (t < lanes)
        for (int64_t f = beg + t; f < end; f += lanes) s += double(x[f]);
    lds[t] = s;
    __syncthreads();
    const int k = t / ncol;
    int half = 1;
    while (2 * half < per) half *= 2;
    for (; half >= 1; half >>= 1) {
        if (t < lanes && k < half && k + half < per) lds[t] += lds[t + half * ncol];
        __syncthreads();
    }
    if (t < ncol) {
        if (parts == 1)
            out[size_t(b) * ncol + t] = float(lds[t]);
        else
            a.part[size_t(z) * a.part_stride + (size_t(b) * parts + p) * ncol + t] = lds[t];
    }
}

// Output q of the energies (q < n_structures) and virials: the sum of its
// parts in part order.
__global__ void k_structure_sum_parts(int n_structures, SumArgs a) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n_structures * 10) return;
    const int z = q < n_structures ? 0 : 1, ncol = z ? 9 : 1;
    const int o = z ? q - n_structures : q;
    float *out = z ? a.d_virial : a.d_energy;
    if (!out) return;
    const int b = o / ncol, c = o - b * ncol;
    const double *part = a.part + size_t(z) * a.part_stride;
    double s = 0.0;
    for (int p = 0; p < a.parts; ++p) s += part[(size_t(b) * a.parts + p) * ncol + c];
    out[o] = float(s);
}

static int sum_parts(const Records &r) {
    return std::max(1, std::min(kMaxSumParts, ceil_div(r.max_struct_atoms, kSumChunk)));
}

}  // namespace

void forces_and_virial(const Records &r, const float4 *g, float *forces, float *atom_virial,
                       hipStream_t s) {
    if (r.n_atoms == 0) return;
    hipLaunchKernelGGL(k_forces, dim3(ceil_div(int64_t(r.n_atoms) * kForceLanes, 256)), dim3(256),
                       0, s, r, g, forces,
                       atom_virial);
    RUNE_HIP_CHECK(hipGetLastError());
}

size_t structure_sum_scratch(const Records &r) {
    const int parts = sum_parts(r);
    return parts == 1 ? 0 : size_t(r.n_structures) * parts * 10;
}

void structure_sums(const Records &r, const float *energies, float *d_energy,
                    const float *atom_virial, float *d_virial, double *scratch, hipStream_t s) {
    if (r.n_structures == 0 || (!d_energy && !d_virial)) return;
    SumArgs a;
    a.energies = energies;
    a.virial = atom_virial;
    a.d_energy = d_energy;
    a.d_virial = d_virial;
    a.parts = sum_parts(r);
    a.part = scratch;
    a.part_stride = size_t(r.n_structures) * a.parts;
    if (a.parts > 1 && !scratch) throw Error(RUNE_ERR_STATE, "structure_sums: no scratch");
    hipLaunchKernelGGL(k_structure_sum, dim3(a.parts, r.n_structures, 2), dim3(1024), 0, s,
                       r.sptr, a);
    if (a.parts > 1)
        hipLaunchKernelGGL(k_structure_sum_parts, dim3(ceil_div(r.n_structures * 10, 256)),
                           dim3(256), 0, s, r.n_structures, a);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
