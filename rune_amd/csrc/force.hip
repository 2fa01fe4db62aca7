// K7: forces and virials from per-record gradients g = dE/dr_ij, without atomics.
//
// F_i = sum_{e: centre i} g_e - sum_{e: neighbour i} g_e   (force.py:151-162,
// model.py:23-44) using the neighbour-grouped transpose list, and the per-atom
// virial W_a = -sum_{e: neighbour a} g_e (x) r_e attributed to the neighbour
// like the reference.  Structure totals use a fixed-order fp64 reduction.
#include "kernels.hpp"

namespace rune {
namespace {

__global__ void k_forces(Records r, const float4 *g, float *forces, float *atom_virial) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= r.n_atoms) return;
    float fx = 0.0f, fy = 0.0f, fz = 0.0f;
    for (int e = r.ptr[i]; e < r.ptr[i + 1]; ++e) {
        float4 v = g[e];
        fx += v.x;
        fy += v.y;
        fz += v.z;
    }
    float w[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int t = r.tptr[i]; t < r.tptr[i + 1]; ++t) {
        int e = r.tidx[t];
        float4 v = g[e];
        fx -= v.x;
        fy -= v.y;
        fz -= v.z;
        if (atom_virial) {
            float4 d = r.vec[e];
            float gv[3] = {v.x, v.y, v.z}, rv[3] = {d.x, d.y, d.z};
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b) w[3 * a + b] -= gv[a] * rv[b];
        }
    }
    if (forces) {
        forces[3 * i + 0] = fx;
        forces[3 * i + 1] = fy;
        forces[3 * i + 2] = fz;
    }
    if (atom_virial)
        for (int k = 0; k < 9; ++k) atom_virial[9 * size_t(i) + k] = w[k];
}

// One workgroup per structure; thread t sums atoms t, t+256, ... then a tree.
__global__ void __launch_bounds__(256) k_structure_sum(const int32_t *sptr, const float *x,
                                                       int ncol, float *out) {
    __shared__ double lds[256];
    int b = blockIdx.x;
    int beg = sptr[b], end = sptr[b + 1];
    for (int c = 0; c < ncol; ++c) {
        double s = 0.0;
        for (int m = beg + threadIdx.x; m < end; m += 256) s += double(x[size_t(m) * ncol + c]);
        lds[threadIdx.x] = s;
        __syncthreads();
        for (int off = 128; off > 0; off >>= 1) {
            if (threadIdx.x < off) lds[threadIdx.x] += lds[threadIdx.x + off];
            __syncthreads();
        }
        if (threadIdx.x == 0) out[size_t(b) * ncol + c] = float(lds[0]);
        __syncthreads();
    }
}

}  // namespace

void forces_and_virial(const Records &r, const float4 *g, float *forces, float *atom_virial,
                       hipStream_t s) {
    if (r.n_atoms == 0) return;
    hipLaunchKernelGGL(k_forces, dim3(ceil_div(r.n_atoms, 256)), dim3(256), 0, s, r, g, forces,
                       atom_virial);
    RUNE_HIP_CHECK(hipGetLastError());
}

void structure_sum(const Records &r, const float *x, int ncol, float *out, hipStream_t s) {
    if (r.n_structures == 0) return;
    hipLaunchKernelGGL(k_structure_sum, dim3(r.n_structures), dim3(256), 0, s, r.sptr, x, ncol,
                       out);
    RUNE_HIP_CHECK(hipGetLastError());
}

}  // namespace rune
