// EQ blocks (rune/mobius/equivariant.py) -- placeholder until the kernels land.
#include "message.hpp"

namespace rune {

void validate_equivariant(ModelImpl &) {
    throw Error(RUNE_ERR_ARGUMENT, "equivariant message blocks are not available in this build");
}
void define_expected_equivariant(ModelImpl &) {}
void pack_equivariant(ModelImpl &, Packer &, std::map<std::string, size_t> &) {}
void bind_equivariant(ModelImpl &, const PackedLookup &) {}
MessagePlan plan_equivariant(ModelImpl &, Arena &, int, int64_t) { return MessagePlan(); }
float *equivariant_forward(ModelImpl &, MessagePlan &, LocalPlan &, const Records &,
                           const int32_t *, const float *, float *h, hipStream_t, bool) {
    return h;
}
float *equivariant_backward(ModelImpl &, MessagePlan &, LocalPlan &, const Records &,
                            const int32_t *, const float *, float *dh, hipStream_t) {
    return dh;
}

}  // namespace rune
