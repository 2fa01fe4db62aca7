// Device-side descriptions of packed model data and kernel launchers.
#pragma once

#include "common.hpp"

namespace rune {

constexpr int kActSigmoid = 3;   // internal activation code next to RUNE_ACT_*

constexpr int kMaxNr = 16;    // radial descriptor channels  (n_max_radial + 1)
constexpr int kMaxKr = 24;    // radial basis size           (basis_size_radial + 1)
constexpr int kMaxNa = 16;    // angular descriptor channels
constexpr int kMaxKa = 24;    // angular basis size
constexpr int kMaxL = 8;      // l_max
constexpr int kMaxLm = kMaxL * (kMaxL + 2);

// Descriptor constants and coefficient tables (device pointers).
struct DescTables {
    int n_types;
    int nr, kr, na, ka, l_max, nlm;
    int num_L, Q;                 // angular invariants per channel, q width
    int has_q[6];                 // q222 q1111 q112 q123 q233 q134
    float rc_r, rc_a;
    int kr4, ka4;                 // kr, ka rounded up to 4: row length of the packed c tables
    const float *c_radial;        // [T,T,nr,kr4], zero past kr
    const float *c_angular;       // [T,T,na,ka4], zero past ka
    const float *z;               // Z_L[n1][p] flattened, offsets z_off[L]
    int z_off[kMaxL + 2];
    const float *c3b;             // [80]
    const float *c4b;             // [5]
    const float *c5b;             // [3]
    const float *c4b2;            // [5]
};

// ZBL (rune/mobius/zbl.py:92-141).
struct ZblTables {
    int mode;                     // RUNE_ZBL_*
    int n_types;
    float rc_inner, rc_outer;
    const float *z;               // atomic numbers [T]
    const float *zpow;            // z^0.23 [T]
    const float *pairs;           // flexible: [T(T+1)/2, 10]
    const float *universal;       // universal (a_k, b_k) pairs [4, 2]
    int on_angular;               // 1: evaluate on the angular list (NEP)
};

// Records of a neighbour list as the kernels see them.
struct Records {
    int n_atoms;
    const int32_t *ptr;           // [N+1]
    const int32_t *view;          // [N,4] rb re ab ae
    const int32_t *nbr;           // [E]
    const float4 *vec;            // [E] {x, y, z, |r|}
    const int32_t *tptr;          // [N+1]
    const int32_t *tidx;          // [E]
    const int32_t *tctr;          // [E] centre of transposed record t
    const int32_t *ctr;           // [E] centre of each record
    const int32_t *sptr;          // [B+1]
    int n_structures;
    const int32_t *order;         // [N] spatially coherent processing order, or null
    int max_struct_atoms;         // atoms of the largest structure
};

// ---- descriptor (descriptor.hip) ----
// n_records (the record count) only steers the launch shape.
void descriptor_forward(const DescTables &t, const Records &r, int64_t n_records,
                        const int32_t *types, float *q, int ldq, float *moments, hipStream_t s);
// dq: [N, ldq]; dmom: [N, na*nlm] or null; g_direct: [E] or null (added);
// energies: ZBL energies added when zbl.mode != NONE; g: [E] output.
void descriptor_reverse(const DescTables &t, const ZblTables &z, const Records &r,
                        int64_t n_records, const int32_t *types, const float *dq, int ldq,
                        const float *moments, const float *dmom, const float4 *g_direct,
                        float *energies, float4 *g, int want_grad, hipStream_t s);

// ---- dense layers (dense.hip) ----
struct Epilogue {
    const float *row_scale = nullptr;   // [M]  v = row_scale[m] * acc
    const float *bias = nullptr;        // [N]
    const float *emb = nullptr;         // [T, ld_emb] added at types[m]
    const int32_t *types = nullptr;
    int ld_emb = 0;
    const float *residual = nullptr;    // [M, ldr]
    int ldr = 0;
    // v += gtab[k][gidx[k][m] * gld[k] + n]   (gathered row adds, k < 3)
    const float *gtab[3] = {nullptr, nullptr, nullptr};
    const int32_t *gidx[3] = {nullptr, nullptr, nullptr};
    int gld[3] = {0, 0, 0};
    float *pre = nullptr;               // store pre-activation [M, ldp]
    int ldp = 0;
    int act = -1;                       // RUNE_ACT_* applied to the output, -1 none
    int act_split = -1;                 // columns >= act_split use act2 instead of act
    int act2 = -1;
    const float *dact_from = nullptr;   // v *= act'(U[m, n]) with U [M, ldu]
    int ldu = 0;
    int dact = -1;                      // activation whose derivative is used
    // RUNE_ACT_* applied to every A element as it is staged (A holds
    // pre-activations), -1 none; the padding of a partial K stage is
    // multiplied by zero B columns, so act(0) there does not matter
    int a_act = -1;
    // RMSNorm of the A rows folded in: when set, v = r[m] * acc with
    // r[m] = 1 / sqrt(mean_k A[m, k]^2 + rms_eps) formed from the rows the
    // GEMM reads (K is the norm width), and r stored to rms_out[m]; used
    // instead of row_scale, not with a_act or batches
    float *rms_out = nullptr;
    float rms_eps = 0.0f;
};
// C[M,N] = A[M,K] Bt[N,K]^T (+ epilogue); row-major with leading dimensions.
void gemm(int M, int N, int K, const float *A, int lda, const float *Bt, int ldb, float *C,
          int ldc, const Epilogue &ep, hipStream_t s);
// count independent products: batch z uses A + z sa, C + z sc and Bt + w sb,
// w = z, or w = L(z) - 1 with L(z) the harmonic order of component z
// (z = L^2 - 1 + m) when b_by_order is set.
struct GemmBatch {
    int count = 1;
    int64_t sa = 0, sb = 0, sc = 0;
    int b_by_order = 0;
};
void gemm_batched(const GemmBatch &bt, int M, int N, int K, const float *A, int lda,
                  const float *Bt, int ldb, float *C, int ldc, hipStream_t s);
// dh[m] = base[m] + r*dz[m] - r^3/N (dz[m].h[m]) h[m]   (RMSNorm backward + residual)
void rms_backward(int M, int N, const float *h, int ldh, const float *inv_rms, const float *dz,
                  int ldz, const float *base, int ldb, float *dh, int ldd, hipStream_t s);
// Möbius readout (layers.py:70-89 on RMSNorm): E = r*(h.hw[t]) + hb[t]; dh = dE/dh.
void readout(int M, int H, const float *h, int ldh, const int32_t *types, const float *hw,
             const float *hb, float eps, float *energies, float *dh, int ldd, hipStream_t s);
// NEP per-element MLP (rune/nep/model.py:157-170): energies and dE/dq.
void nep_mlp(int M, int Q, int Hn, const float *q, int ldq, const int32_t *types,
             const float *w0, const float *b0, const float *w1, float shared_bias,
             float *energies, float *dq, int want_grad, hipStream_t s);

// ---- forces (force.hip) ----
void forces_and_virial(const Records &r, const float4 *g, float *forces, float *atom_virial,
                       hipStream_t s);
// Per-structure sums of the per-atom energies (one column) and virials
// (nine columns): d_energy[b] and d_virial[b, c] over the atoms of structure
// b, fp64 accumulation in a fixed order for a given structure layout; a null
// output is skipped.  Structures larger than kSumChunk atoms are split over
// up to kMaxSumParts blocks whose fp64 partials go to scratch, combined in
// part order; structure_sum_scratch(r) doubles are needed (0: none).
constexpr int kSumChunk = 1024, kMaxSumParts = 256;
struct SumArgs {
    const float *energies = nullptr, *virial = nullptr;
    float *d_energy = nullptr, *d_virial = nullptr;
    int parts = 1;
    double *part = nullptr;
    size_t part_stride = 0;   // doubles per output's partials (n_structures * parts)
};
size_t structure_sum_scratch(const Records &r);
void structure_sums(const Records &r, const float *energies, float *d_energy,
                    const float *atom_virial, float *d_virial, double *scratch, hipStream_t s);

}  // namespace rune
