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

struct ResidualWeights {
    const float *w1, *w1T, *b1, *w2, *w2T, *b2;
};

// Weights of one message block (MP: message.py, EQ: equivariant.py), packed.
struct MessageWeights {
    const float *in_norm;       // [H]
    const float *pair_emb;      // [T*T, P]
    const float *edge_w;        // edge MLP weight rows [D, K_edge]  (radial|pair part)
    const float *edge_wT;       // [K_edge, D]
    const float *edge_b;        // [D]
    const float *gate_w;        // group gate [G, D]
    const float *gate_b;        // [G]
    const float *value_wT;      // [H, H] value projection^T  (W_v^T)
    const float *value_w;       // [H, H]
    // MP vector branch
    const float *vgate_w, *vgate_b;   // [vc, D], [vc]
    const float *vsrc_wT, *vsrc_w;    // [H, vc], [vc, H]
    const float *vmix;                // [vc, vc]
    // EQ
    const float *ctx_wT, *ctx_w;      // [H, 2D] (centre | neighbour contexts), [2D, H]
    const float *dir_w, *dir_b;       // direction gates [2*lq*C, D], [2*lq*C]
    const float *mix;                 // [lq, C, C]
    const float *edge_w_ctx;          // edge MLP columns acting on probes [D, 2*lq*C]
    // update MLP
    const float *msg_norm;            // [H]
    const float *up1_w, *up1_wT, *up1_b;   // [D, H+X], [H+X, D], [D]
    const float *up2_w, *up2_wT, *up2_b;   // [H, D], [D, H], [H]
    const float *pair_proj;           // EQ: pair_emb @ W_pair^T + b  [T*T, D]
};

struct LocalPlan {
    size_t o_h = 0, o_r = 0, o_u = 0, o_a = 0, o_dha = 0, o_dhb = 0, o_dz = 0;
    int N = 0, H = 0, F = 0;
    float *h = nullptr, *r = nullptr, *u = nullptr, *a = nullptr;
    float *dh_a = nullptr, *dh_b = nullptr, *dz = nullptr;
    void bind(char *base);
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
    void bind(char *base);
    float *at(int k) const { return ptrs[k]; }
};

struct ModelImpl {
    rune_model_config cfg{};
    std::vector<std::string> elements;
    int Q = 0;
    std::map<std::string, int64_t> expected;
    std::map<std::string, std::vector<float>> host;
    bool finalized = false;
    DeviceBuffer weights;
    DeviceBuffer work;
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
    // phase timing ring (events recorded on the launch stream)
    bool timing = false;
    std::vector<hipEvent_t> events;       // kTimingRing x (RUNE_N_PHASES + 1)
    int64_t timed_calls = 0;
    const std::vector<float> &tensor(const std::string &name) const;
    ~ModelImpl();
};

constexpr int kTimingRing = 256;

using PackedLookup = std::function<const float *(const std::string &)>;

// message.hip
void validate_messages(ModelImpl &m);
void define_expected_messages(ModelImpl &m);
void pack_messages(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off);
void bind_messages(ModelImpl &m, const PackedLookup &P);
MessagePlan plan_messages(ModelImpl &m, Arena &ar, int N, int64_t E);
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
