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
// Block (p, b) takes part p of structure b's atoms (one part unless the
// structure is large) and reads them as one flat coalesced range; the
// threads in use are a multiple of ncol, so thread t always meets column
// t % ncol.  The per-thread partials of each column are combined by a fixed
// tree.  With one part the result goes to out, else to part[b, p, :].
__global__ void __launch_bounds__(1024) k_structure_sum(const int32_t *sptr, const float *x,
                                                        int ncol, int parts, double *part,
                                                        float *out) {
    __shared__ double lds[1024];
    const int b = blockIdx.y, p = blockIdx.x, t = threadIdx.x;
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
            part[(size_t(b) * parts + p) * ncol + t] = lds[t];
    }
}

// out[b, c] = sum of the parts of structure b in part order.
__global__ void k_structure_sum_parts(int n_structures, int ncol, int parts, const double *part,
                                      float *out) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n_structures * ncol) return;
    const int b = q / ncol, c = q - b * ncol;
    double s = 0.0;
    for (int p = 0; p < parts; ++p) s += part[(size_t(b) * parts + p) * ncol + c];
    out[q] = float(s);
}

static int sum_parts(const Records &r) {
    return std::max(1, std::min(64, ceil_div(r.max_struct_atoms, kSumChunk)));
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

size_t structure_sum_scratch(const Records &r, int ncol) {
    const int parts = sum_parts(r);
    return parts == 1 ? 0 : size_t(r.n_structures) * parts * ncol;
}

void structure_sum(const Records &r, const float *x, int ncol, float *out, double *scratch,
                   hipStream_t s) {
    if (r.n_structures == 0) return;
    if (ncol < 1 || ncol > 1024) throw Error(RUNE_ERR_ARGUMENT, "structure_sum: bad column count");
    const int parts = sum_parts(r);
    if (parts > 1 && !scratch) throw Error(RUNE_ERR_STATE, "structure_sum: no scratch");
    hipLaunchKernelGGL(k_structure_sum, dim3(parts, r.n_structures), dim3(1024), 0, s, r.sptr, x,
                       ncol, parts, scratch, out);
    if (parts > 1)
        hipLaunchKernelGGL(k_structure_sum_parts, dim3(ceil_div(r.n_structures * ncol, 256)),
                           dim3(256), 0, s, r.n_structures, ncol, parts, scratch, out);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
