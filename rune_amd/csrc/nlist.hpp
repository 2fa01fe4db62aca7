// Internal layout of a neighbour-list handle (shared by the model code).
#pragma once

#include "common.hpp"

struct rune_nlist {
    int64_t n_atoms = 0;
    int64_t n_records = 0;
    int32_t n_structures = 0;
    double rc_radial = 0.0, rc_angular = 0.0;
    bool from_padded = false;
    std::vector<int64_t> h_struct_ptr;   // host copy of structure ranges

    // records (see include/rune_hip.h)
    rune::DeviceBuffer ptr;      // int32 [N+1]
    rune::DeviceBuffer view;     // int32 [N,4] {rb, re, ab, ae}
    rune::DeviceBuffer nbr;      // int32 [E]
    rune::DeviceBuffer shift;    // int32 [E,3]
    rune::DeviceBuffer vec;      // float4 [E]
    rune::DeviceBuffer ctr;      // int32 [E] centre atom of each record
    // transpose: records whose neighbour is atom a, ascending record id
    rune::DeviceBuffer tptr;     // int32 [N+1]
    rune::DeviceBuffer tidx;     // int32 [E]
    rune::DeviceBuffer tctr;     // int32 [E] centre of each transposed record
    rune::DeviceBuffer sptr;     // int32 [B+1] device copy of structure ranges
    rune::DeviceBuffer geo;      // bin frames of the structures
    rune::DeviceBuffer perm;     // int32 Morton rank of every bin
    // host copies of what sptr, geo and perm last received (repeated builds of
    // one system upload nothing), and the bin grids behind h_perm
    std::vector<char> sptr_shadow, geo_shadow, perm_shadow, perm_geo;
    // atoms in cell-bin order (spatially coherent processing order); empty
    // for lists made from padded tensors
    rune::DeviceBuffer order;    // int32 [N]
    bool has_order = false;
    // whether the last model that read this list walks atoms in the processing
    // order (the message blocks do; the descriptor and force kernels do not):
    // a build computes the order only then (without it the walks take index
    // order, with identical results)
    mutable bool order_wanted = true;
    std::vector<int32_t> h_perm; // host Morton ranks of the bins
    // skin reuse (rune_nlist_update): candidates within max(rc) + skin of the
    // last search, the positions it saw, and what else it depended on
    rune::DeviceBuffer cand_keys;   // uint64 [N, cand_cap], sorted per centre
    rune::DeviceBuffer cand_cnt;    // int32 [N]
    rune::DeviceBuffer ref_pos;     // fp64 [N, 3]
    rune::DeviceBuffer cand_flag;   // int32 displacement flag
    int cand_cap = 0;
    bool cand_valid = false;
    std::vector<double> cand_key;
    // working memory of the builder
    rune::DeviceBuffer work;
    rune::DeviceBuffer extent;   // bin frames and atom extents of open directions
    rune::DeviceBuffer keys;     // uint64 [N, max(max_radial, max_angular)] sorted per centre
    rune::DeviceBuffer pinned_dummy;
    rune::PinnedWords readback;  // record total and flags of the last build
};

namespace rune {
// Exclusive scan of n int32 values: out[0..n] with out[n] = total.
// tmp must hold scan_tmp_ints(n) ints.
size_t scan_tmp_ints(int64_t n);
void exclusive_scan(const int32_t *in, int32_t *out, int64_t n, int32_t *tmp, hipStream_t s);
}  // namespace rune
