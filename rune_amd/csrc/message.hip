// Message blocks: MP (rune/mobius/message.py) and EQ (rune/mobius/equivariant.py).
#include "model.hpp"

namespace rune {

void MessagePlan::bind(char *base) {
    ptrs.clear();
    for (size_t o : offs) ptrs.push_back(reinterpret_cast<float *>(base + o));
    if (E > 0 || N > 0) {
        g_direct = reinterpret_cast<float4 *>(base + o_gd);
        dmom = reinterpret_cast<float *>(base + o_dmom);
    }
}

void validate_messages(ModelImpl &m) {
    if (m.cfg.family != RUNE_FAMILY_MOBIUS || m.cfg.message_layers == 0) return;
    throw Error(RUNE_ERR_ARGUMENT, "message blocks are not available in this build yet");
}

void define_expected_messages(ModelImpl &) {}

void pack_messages(ModelImpl &, Packer &, std::map<std::string, size_t> &) {}

void bind_messages(ModelImpl &, const PackedLookup &) {}

MessagePlan plan_messages(ModelImpl &, Arena &, int N, int64_t E) {
    MessagePlan p;
    p.N = 0;
    p.E = 0;
    (void)N;
    (void)E;
    return p;
}

float *messages_forward(ModelImpl &, MessagePlan &, LocalPlan &, const Records &,
                        const int32_t *, const float *, float *h, hipStream_t, bool) {
    return h;
}

float *messages_backward(ModelImpl &, MessagePlan &, LocalPlan &, const Records &,
                         const int32_t *, const float *, float *dh, hipStream_t) {
    return dh;
}

}  // namespace rune
