// Declarations shared by the MP (message.hip) and EQ (equivariant.hip) blocks.
#pragma once

#include "model.hpp"

namespace rune {

struct EdgePrepArgs {
    Records r;
    int64_t E;
    const int32_t *types;
    int n_types;
    float cutoff;          // message_cutoff
    int kb, ldrb;          // message basis size, row stride of rb
    float *rb;             // [E, ldrb] masked Chebyshev basis (message.py:108-110)
    float *rbd;            // [E, ldrb] its derivative with respect to the distance, or null
    float *fc;             // [E] cosine cutoff, 0 outside the radial list
    int32_t *pair;         // [E] t_i * T + t_j
    float4 *dv;            // [E] zeroed: (dE/du, dE/dd) accumulators
    float *dd;             // [E] zeroed second dE/dd accumulator, or null
    float *harm;           // EQ: [E, nq] normalised harmonics, or null
    const float *scale;    // [nq] orthonormal scale
    int lq, nq;
    const float *z;        // Z tables (flattened) and offsets
    int z_off[kMaxL + 2];
};

// Real harmonics of order 1..lq at the unit vector (x, y, z), times scale:
// the polynomial basis of descriptor.py:574-624 with Z tables z.
__device__ inline void harmonics(const float *ztab, const int *z_off, int lq, float x, float y,
                                 float z, const float *scale, float *out) {
    float zp[kMaxL + 1], wr[kMaxL + 1], wi[kMaxL + 1];
    zp[0] = 1.0f;
    wr[0] = 1.0f;
    wi[0] = 0.0f;
    for (int k = 1; k <= lq; ++k) {
        zp[k] = zp[k - 1] * z;
        wr[k] = wr[k - 1] * x - wi[k - 1] * y;
        wi[k] = wr[k - 1] * y + wi[k - 1] * x;
    }
    int idx = 0;
    for (int L = 1; L <= lq; ++L) {
        for (int n1 = 0; n1 <= L; ++n1) {
            const float *Z = ztab + z_off[L] + n1 * (L + 1);
            float zf = 0.0f;
            for (int q = ((L + n1) & 1); q <= L - n1; q += 2) zf += Z[q] * zp[q];
            if (n1 == 0) {
                out[idx] = zf * scale[idx];
                ++idx;
            } else {
                out[idx] = zf * wr[n1] * scale[idx];
                ++idx;
                out[idx] = zf * wi[n1] * scale[idx];
                ++idx;
            }
        }
    }
}

// Host helpers (message.hip)
std::vector<float> fold_cols(const std::vector<float> &w, int rows, int cols, const float *s);
std::vector<float> columns(const std::vector<float> &w, int rows, int cols, int c0, int c1);
std::vector<float> pair_projection(const std::vector<float> &emb, const std::vector<float> &w,
                                   const std::vector<float> &b, int TT, int P, int D, int K,
                                   int c0);
void edge_prep(ModelImpl &m, MessagePlan &p, const Records &r, const int32_t *types,
               hipStream_t s, float *harm, const float *scale, int lq, int nq);
void edge_rb_backward(ModelImpl &m, MessagePlan &p, const Records &r, const float *drb, int ld,
                      hipStream_t s);

struct EdgeZ {
    int off[kMaxL + 2];
};
void edge_direct(MessagePlan &p, const Records &r, hipStream_t s);

// EQ (equivariant.hip)
void validate_equivariant(ModelImpl &m);
void define_expected_equivariant(ModelImpl &m);
void pack_equivariant(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off);
void bind_equivariant(ModelImpl &m, const PackedLookup &P);
MessagePlan plan_equivariant(ModelImpl &m, Arena &ar, int N, int64_t E);
void equivariant_record_forward(ModelImpl &m, MessagePlan &p, const Records &r,
                                const int32_t *types, hipStream_t s);
float *equivariant_forward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                           const int32_t *types, const float *moments, float *h, hipStream_t s,
                           bool keep);
float *equivariant_backward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                            const int32_t *types, const float *moments, float *dh,
                            hipStream_t s);

}  // namespace rune
