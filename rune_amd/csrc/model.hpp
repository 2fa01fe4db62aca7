// Internal model structure shared by model.hip and the message-block code.
#pragma once

#include <functional>
#include <map>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "nlist.hpp"

namespace rune {

const char *g_last_error_ptr();

struct Packer {
    std::vector<float> data;
    size_t put(const float *p, size_t n);
    size_t put(const std::vector<float> &v);
};

std::vector<float> transpose(const std::vector<float> &w, int rows, int cols);
// W [rows, cols] -> [rows, (cols + 3) & ~3], zero columns appended (16-byte rows).
std::vector<float> pad_rows(const std::vector<float> &w, int rows, int cols);

struct ResidualWeights {
    const float *w1, *w1T, *b1, *w2, *w2T, *b2;
};

// Weights of one message block (MP: message.py, EQ: equivariant.py), packed.
// "f" = RMSNorm weight folded into the columns.  The GEMM takes its weight
// operand as Bt[N, K] (K contiguous): the [out, in] copy serves the forward
// products and the "T" (transposed, [in, out]) copy the reverse ones.
struct MessageWeights {
    // node projections of RMSNorm(h):  MP [values | vector source],
    // EQ [W_e,c C_c | W_e,n C_n | values]
    const float *node_fT, *node_f;    // [H, NP], [NP, H]
    int NP;
    // edge MLP on per-edge features: MP [radial basis], EQ [radial basis | probes]
    const float *edge_xT, *edge_x;    // [KX, D], [D, ld_edge_x]
    int KX, ld_edge_x;
    // EQ factored edge MLP: radial-basis rows [kb, D], probe rows [lq*C, D],
    // both probe blocks per order [lq][C][2 ldd] (zero past D), and the gate
    // transpose with zero rows up to ldd [ldd, NG]
    const float *edge_rbT = nullptr, *probe_c = nullptr, *probe_n = nullptr;
    const float *probe_cat = nullptr, *gate_Tp = nullptr;
    const float *pair_proj;           // [T*T, D] = pair_embedding W_pair^T + b
    // gates from the edge hidden state: MP [groups | vector], EQ [groups | directions]
    const float *gate_T, *gate, *gate_b;   // [D, NG], [NG, D], [NG]
    int NG;
    const float *vmix;                // MP [vc, vc]
    const float *mix;                 // EQ [lq, C, C]
    // update MLP on [RMSNorm(message) | invariants]
    const float *up1_fT, *up1_f, *up1_b;   // [H+X, D], [D, H+X], [D]
    const float *up2_T, *up2, *up2_b;      // [D, H], [H, D], [H]
};

struct LocalPlan {
    size_t o_h = 0, o_r = 0, o_u = 0, o_a = 0, o_dha = 0, o_dhb = 0, o_dz = 0;
    int N = 0, H = 0, F = 0;
    float *h = nullptr, *r = nullptr, *u = nullptr, *a = nullptr;
    float *dh_a = nullptr, *dh_b = nullptr, *dz = nullptr;
    void bind(char *base);
};

// Workspace indices of one message block (entries of MessagePlan::offs).
struct BlockBuffers {
    int h_out = -1, rin = -1, vs = -1, ue = -1, eh = -1, gv = -1, msg = -1, rm = -1;
    int vsum = -1, mixed = -1, uin = -1, u1 = -1, z1 = -1;
    int dir_in = -1, dir_out = -1, mixstate = -1;   // EQ angular states
    int q = -1;                                      // EQ per-atom edge-MLP factors
    int dgv = -1;   // MP: this block's gate adjoints, when its edge reverse runs on the side stream
};

struct MessagePlan {
    std::vector<size_t> offs;
    std::vector<float *> ptrs;
    float4 *g_direct = nullptr;
    float *dmom = nullptr;
    bool g_direct_used = false, dmom_used = false;
    int N = 0;
    int64_t E = 0;
    size_t o_gd = 0, o_dmom = 0;
    int ldrb = 0;
    int ld_edge = 0;              // EQ: row stride of the per-record [E, D] arrays
    bool records_ready = false;   // record-only forward work already enqueued (side stream)
    int i_dd = -1;                // MP: [E] dE/dd of the edge reverses run on the side stream
    int i_rb = -1, i_fc = -1, i_tfc = -1, i_pair = -1, i_dv = -1, i_harm = -1, i_dharm = -1, i_zero = -1;
    int i_dfc = -1, i_drb = -1, i_rbd = -1;
    std::vector<BlockBuffers> blocks;
    // reverse-pass temporaries shared by the blocks
    int t_dz1 = -1, t_duin = -1, t_dmsg = -1, t_dvsum = -1, t_dgv = -1, t_due = -1;
    int t_drb = -1, t_dvs = -1, t_dz = -1, t_dh0 = -1, t_dh1 = -1;
    int t_ddir0 = -1, t_ddir1 = -1, t_dmix = -1, t_dab = -1;
    int t_dq = -1, t_dhk = -1;    // EQ: per-atom factor adjoints, their channel projection
    std::vector<const float *> block_input;
    int add(Arena &ar, size_t bytes);
    void bind(char *base);
    float *at(int k) const { return ptrs[k]; }
};

struct ModelImpl {
    rune_model_config cfg{};
    std::vector<std::string> elements;
    // neighbour limits from a text artifact (0 when created from a config)
    int max_radial = 0, max_angular = 0;
    int Q = 0;
    std::map<std::string, int64_t> expected;
    std::map<std::string, std::vector<float>> host;
    bool finalized = false;
    DeviceBuffer weights;
    DeviceBuffer work;
    DeviceBuffer sums;        // fp64 partial sums of the split structure reductions
    DeviceBuffer gpumd_out;   // fp32 energies, forces, atom virial of rune_model_compute_gpumd
    DescTables desc{};
    ZblTables zbl{};
    // Möbius local network
    const float *in_w = nullptr, *in_wT = nullptr, *in_b = nullptr, *emb = nullptr;
    std::vector<ResidualWeights> res;
    const float *head_w = nullptr, *head_b = nullptr;
    std::vector<MessageWeights> msg;
    const float *enc_w = nullptr;     // EQ direction encoder [lq, C, na] (scaled)
    const float *harm_scale = nullptr;  // orthonormal scale [nlm_q]
    // NEP
    const float *nep_w0 = nullptr, *nep_b0 = nullptr, *nep_w1 = nullptr;
    float nep_bias = 0.0f;
    // type-check verdict: pinned host word written behind the check kernel,
    // and the event that marks its arrival (created by rune_model_finalize)
    int32_t *type_flag_host = nullptr;
    hipEvent_t type_event = nullptr;
    bool type_pending = false;   // type_event recorded, verdict not yet read
    // side stream (default priority) for the record-only work of the message
    // blocks, forked from and joined back into the launch stream by events
    hipStream_t side = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    // phase timing ring (events recorded on the launch stream)
    int timing = 0;   // 0 off, 1 phase events and kernel-group spans, 2 spans only
    std::vector<hipEvent_t> events;       // kTimingRing x (RUNE_N_PHASES + 1)
    int64_t timed_calls = 0;
    // kernel-group spans: events 2k, 2k + 1 bracket launch k of group span_grp[k]
    std::vector<hipEvent_t> span_ev;
    std::vector<int> span_grp;
    size_t span_n = 0;
    int span_begin(int group, hipStream_t s);
    void span_end(int k, hipStream_t s);
    const std::vector<float> &tensor(const std::string &name) const;
    ~ModelImpl();
};

constexpr int kTimingRing = 256;
constexpr size_t kMaxSpans = 1 << 16;

// Brackets the launches issued in its scope with a group span (no-op unless
// timing is enabled).
struct Span {
    ModelImpl &m;
    hipStream_t s;
    int k;
    Span(ModelImpl &model, int group, hipStream_t stream)
        : m(model), s(stream), k(model.span_begin(group, stream)) {}
    ~Span() { m.span_end(k, s); }
    Span(const Span &) = delete;
    Span &operator=(const Span &) = delete;
};

using PackedLookup = std::function<const float *(const std::string &)>;

// message.hip
void validate_messages(ModelImpl &m);
void define_expected_messages(ModelImpl &m);
void pack_messages(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off);
void bind_messages(ModelImpl &m, const PackedLookup &P);
MessagePlan plan_messages(ModelImpl &m, Arena &ar, int N, int64_t E);
// Enqueues the message blocks' record-only forward work (no node state read)
// on m.side after an event on s; false when the model has none to move.
bool messages_records_ahead(ModelImpl &m, MessagePlan &p, const Records &r,
                            const int32_t *types, hipStream_t s);
float *messages_forward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                        const int32_t *types, const float *moments, float *h, hipStream_t s,
                        bool keep);
float *messages_backward(ModelImpl &m, MessagePlan &p, LocalPlan &lp, const Records &r,
                         const int32_t *types, const float *moments, float *dh, hipStream_t s);

// model.hip
LocalPlan plan_local(ModelImpl &m, Arena &ar, int N);
float *local_forward(ModelImpl &m, LocalPlan &p, int N, const float *q, int ldq,
                     const int32_t *types, hipStream_t s);
void local_backward(ModelImpl &m, LocalPlan &p, int N, float *dh, float *dq, int ldq,
                    hipStream_t s);

}  // namespace rune

// The C-ABI handle (include/rune_hip.h).
struct rune_model : rune::ModelImpl {};
