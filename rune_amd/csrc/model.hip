// Model handle: weight packing and the forward / reverse schedule.
//
// Schedule of one call (Mobius.forward, rune/mobius/model.py:307-393):
//   K2 descriptor forward          q, moments
//   input projection + residual    h_0 .. h_B            (MFMA GEMMs)
//   message blocks (MP / EQ)       h, angular states
//   readout                        E_i and dE/dh
//   reverse of the above           dE/dq (+ dE/dmoments, direct dE/dr_ij)
//   K3 descriptor reverse + ZBL    g_e = dE/dr_e per record
//   K7 forces, per-atom virials, structure totals
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>

#include "model.hpp"

namespace rune {

namespace {
thread_local std::string g_last_error;

std::string str(const char *p) { return p ? std::string(p) : std::string(); }
}  // namespace

void set_last_error(const std::string &msg) { g_last_error = msg; }

const char *g_last_error_ptr() { return g_last_error.c_str(); }

// ---------------------------------------------------------------------------
// expected state_dict entries
// ---------------------------------------------------------------------------

static void expect(ModelImpl &m, const std::string &name, int64_t n) { m.expected[name] = n; }

static void define_expected(ModelImpl &m) {
    const rune_model_config &c = m.cfg;
    const int64_t T = c.n_types;
    expect(m, "q_scaler", m.Q);
    expect(m, "descriptor.radial.c_table", T * T * c.n_desc_radial * c.k_radial);
    expect(m, "descriptor.angular.c_table", T * T * c.n_desc_angular * c.k_angular);
    expect(m, "descriptor.angular.C3B", 80);
    expect(m, "descriptor.angular.C4B", 5);
    expect(m, "descriptor.angular.C5B", 3);
    expect(m, "descriptor.angular.C4B2", 5);
    for (int L = 1; L <= 8; ++L) expect(m, "descriptor.angular.Z" + std::to_string(L), (L + 1) * (L + 1));
    if (c.zbl_mode != RUNE_ZBL_NONE) {
        expect(m, "zbl.atomic_numbers", T);
        expect(m, "zbl.universal_coefficients", 8);
        expect(m, "zbl.pair_parameters", c.zbl_mode == RUNE_ZBL_FLEXIBLE ? T * (T + 1) / 2 * 10 : 0);
    }
    if (c.family == RUNE_FAMILY_NEP) {
        for (int t = 0; t < T; ++t) {
            std::string p = "element_mlps." + m.elements[t] + ".";
            expect(m, p + "0.weight", int64_t(c.nep_hidden) * m.Q);
            expect(m, p + "0.bias", c.nep_hidden);
            expect(m, p + "2.weight", c.nep_hidden);
        }
        expect(m, "shared_bias", 1);
        return;
    }
    const int64_t H = c.hidden_dim, F = c.ffn_dim;
    expect(m, "input_projection.weight", H * m.Q);
    expect(m, "input_projection.bias", H);
    expect(m, "element_embedding.weight", T * H);
    for (int b = 0; b < c.blocks; ++b) {
        std::string p = "residual_blocks." + std::to_string(b) + ".";
        expect(m, p + "norm.weight", H);
        expect(m, p + "ffn.0.weight", F * H);
        expect(m, p + "ffn.0.bias", F);
        expect(m, p + "ffn.2.weight", H * F);
        expect(m, p + "ffn.2.bias", H);
    }
    expect(m, "output_norm.weight", H);
    expect(m, "energy_heads.weight", T * H);
    expect(m, "energy_heads.bias", T);
    define_expected_messages(m);
}

// ---------------------------------------------------------------------------
// packing
// ---------------------------------------------------------------------------

size_t Packer::put(const float *p, size_t n) {
    size_t off = data.size();
    data.insert(data.end(), p, p + n);
    while (data.size() % 64) data.push_back(0.0f);
    return off;
}

size_t Packer::put(const std::vector<float> &v) { return put(v.data(), v.size()); }

const std::vector<float> &ModelImpl::tensor(const std::string &name) const {
    auto it = host.find(name);
    if (it == host.end()) throw Error(RUNE_ERR_STATE, "missing tensor " + name);
    return it->second;
}

// W [rows, cols] -> W^T [cols, rows]
std::vector<float> transpose(const std::vector<float> &w, int rows, int cols) {
    std::vector<float> t(size_t(rows) * cols);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) t[size_t(c) * rows + r] = w[size_t(r) * cols + c];
    return t;
}

std::vector<float> pad_rows(const std::vector<float> &w, int rows, int cols) {
    const int ld = (cols + 3) & ~3;
    std::vector<float> t(size_t(rows) * ld, 0.0f);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) t[size_t(r) * ld + c] = w[size_t(r) * cols + c];
    return t;
}

static void pack_descriptor(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off) {
    const rune_model_config &c = m.cfg;
    // c tables with each (t1, t2, n) row padded with zeros to a multiple of 4,
    // so the descriptor kernels read them as 16-byte vectors
    auto padded = [](const std::vector<float> &t, int k, int k4) {
        const size_t rows = t.size() / size_t(k);
        std::vector<float> out(rows * k4, 0.0f);
        for (size_t r = 0; r < rows; ++r)
            std::copy(t.begin() + r * k, t.begin() + (r + 1) * k, out.begin() + r * k4);
        return out;
    };
    m.desc.kr4 = (c.k_radial + 3) & ~3;
    m.desc.ka4 = (c.k_angular + 3) & ~3;
    off["c_radial"] = pk.put(padded(m.tensor("descriptor.radial.c_table"), c.k_radial, m.desc.kr4));
    off["c_angular"] =
        pk.put(padded(m.tensor("descriptor.angular.c_table"), c.k_angular, m.desc.ka4));
    std::vector<float> z;
    int zo = 0;
    for (int L = 1; L <= 8; ++L) {
        m.desc.z_off[L] = zo;
        const auto &t = m.tensor("descriptor.angular.Z" + std::to_string(L));
        z.insert(z.end(), t.begin(), t.end());
        zo += int(t.size());
    }
    off["z"] = pk.put(z);
    off["c3b"] = pk.put(m.tensor("descriptor.angular.C3B"));
    off["c4b"] = pk.put(m.tensor("descriptor.angular.C4B"));
    off["c5b"] = pk.put(m.tensor("descriptor.angular.C5B"));
    off["c4b2"] = pk.put(m.tensor("descriptor.angular.C4B2"));
    if (c.zbl_mode != RUNE_ZBL_NONE) {
        const auto &zn = m.tensor("zbl.atomic_numbers");
        std::vector<float> zp(zn.size());
        for (size_t t = 0; t < zn.size(); ++t) zp[t] = std::pow(zn[t], 0.23f);
        off["zbl_z"] = pk.put(zn);
        off["zbl_zpow"] = pk.put(zp);
        off["zbl_universal"] = pk.put(m.tensor("zbl.universal_coefficients"));
        const auto &pp = m.tensor("zbl.pair_parameters");
        off["zbl_pairs"] = pk.put(pp.empty() ? std::vector<float>(10, 0.0f) : pp);
    }
}

static void pack_local(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off) {
    const rune_model_config &c = m.cfg;
    const int H = c.hidden_dim, F = c.ffn_dim, Q = m.Q, T = c.n_types;
    const auto &qs = m.tensor("q_scaler");
    // input projection with the descriptor scaler folded in: W'[h, q] = W[h, q] * s[q]
    std::vector<float> win = m.tensor("input_projection.weight");
    for (int h = 0; h < H; ++h)
        for (int q = 0; q < Q; ++q) win[size_t(h) * Q + q] *= qs[q];
    off["in_w"] = pk.put(win);                       // [H, Q]  (reverse: B = W')
    off["in_wT"] = pk.put(transpose(win, H, Q));     // [Q, H]
    off["in_b"] = pk.put(m.tensor("input_projection.bias"));
    off["emb"] = pk.put(m.tensor("element_embedding.weight"));
    for (int b = 0; b < c.blocks; ++b) {
        std::string p = "residual_blocks." + std::to_string(b) + ".";
        const auto &wn = m.tensor(p + "norm.weight");
        std::vector<float> w1 = m.tensor(p + "ffn.0.weight");  // [F, H], fold norm weight
        for (int f = 0; f < F; ++f)
            for (int h = 0; h < H; ++h) w1[size_t(f) * H + h] *= wn[h];
        const auto &w2 = m.tensor(p + "ffn.2.weight");        // [H, F]
        off[p + "w1"] = pk.put(w1);
        off[p + "w1T"] = pk.put(transpose(w1, F, H));
        off[p + "b1"] = pk.put(m.tensor(p + "ffn.0.bias"));
        off[p + "w2"] = pk.put(w2);
        off[p + "w2T"] = pk.put(transpose(w2, H, F));
        off[p + "b2"] = pk.put(m.tensor(p + "ffn.2.bias"));
    }
    std::vector<float> hw = m.tensor("energy_heads.weight");  // [T, H] * output_norm.weight
    const auto &wo = m.tensor("output_norm.weight");
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < H; ++h) hw[size_t(t) * H + h] *= wo[h];
    off["head_w"] = pk.put(hw);
    off["head_b"] = pk.put(m.tensor("energy_heads.bias"));
}

static void pack_nep(ModelImpl &m, Packer &pk, std::map<std::string, size_t> &off) {
    const int T = m.cfg.n_types, Hn = m.cfg.nep_hidden, Q = m.Q;
    const auto &qs = m.tensor("q_scaler");
    std::vector<float> w0, b0, w1;
    for (int t = 0; t < T; ++t) {
        std::string p = "element_mlps." + m.elements[t] + ".";
        std::vector<float> w = m.tensor(p + "0.weight");
        for (int h = 0; h < Hn; ++h)
            for (int q = 0; q < Q; ++q) w[size_t(h) * Q + q] *= qs[q];
        w0.insert(w0.end(), w.begin(), w.end());
        const auto &b = m.tensor(p + "0.bias");
        b0.insert(b0.end(), b.begin(), b.end());
        const auto &o = m.tensor(p + "2.weight");
        w1.insert(w1.end(), o.begin(), o.end());
    }
    off["nep_w0"] = pk.put(w0);
    off["nep_b0"] = pk.put(b0);
    off["nep_w1"] = pk.put(w1);
    m.nep_bias = m.tensor("shared_bias")[0];
}

static void finalize(ModelImpl &m) {
    for (const auto &kv : m.expected)
        if (!m.host.count(kv.first))
            throw Error(RUNE_ERR_STATE, "missing state_dict tensor " + kv.first);
    Packer pk;
    std::map<std::string, size_t> off;
    pack_descriptor(m, pk, off);
    if (m.cfg.family == RUNE_FAMILY_NEP) {
        pack_nep(m, pk, off);
    } else {
        pack_local(m, pk, off);
        pack_messages(m, pk, off);
    }
    m.weights.reserve(pk.data.size() * sizeof(float));
    RUNE_HIP_CHECK(hipMemcpy(m.weights.ptr, pk.data.data(), pk.data.size() * sizeof(float),
                             hipMemcpyHostToDevice));
    if (!m.type_flag_host) {
        void *flag = nullptr;
        RUNE_HIP_CHECK(hipHostMalloc(&flag, 64, hipHostMallocCoherent));
        m.type_flag_host = static_cast<int32_t *>(flag);
        *m.type_flag_host = 0;
    }
    if (!m.type_event) RUNE_HIP_CHECK(hipEventCreateWithFlags(&m.type_event, hipEventDisableTiming));
    // the side stream serves the MP blocks (EQ keeps one stream: overlapping
    // its heavier record kernels gained 0.3 % and stretched their durations)
    if (!m.side && m.cfg.family == RUNE_FAMILY_MOBIUS && m.cfg.message_layers > 0 &&
        m.cfg.message_mode != RUNE_MESSAGE_EQUIVARIANT) {
        RUNE_HIP_CHECK(hipStreamCreateWithFlags(&m.side, hipStreamNonBlocking));
        RUNE_HIP_CHECK(hipEventCreateWithFlags(&m.fork_ev, hipEventDisableTiming));
        RUNE_HIP_CHECK(hipEventCreateWithFlags(&m.join_ev, hipEventDisableTiming));
    }
    const float *base = m.weights.as<float>();
    auto P = [&](const std::string &k) -> const float * {
        auto it = off.find(k);
        if (it == off.end()) throw Error(RUNE_ERR_STATE, "internal: no packed " + k);
        return base + it->second;
    };
    DescTables &d = m.desc;
    d.c_radial = P("c_radial");
    d.c_angular = P("c_angular");
    d.z = P("z");
    d.c3b = P("c3b");
    d.c4b = P("c4b");
    d.c5b = P("c5b");
    d.c4b2 = P("c4b2");
    ZblTables &z = m.zbl;
    if (m.cfg.zbl_mode != RUNE_ZBL_NONE) {
        z.z = P("zbl_z");
        z.zpow = P("zbl_zpow");
        z.universal = P("zbl_universal");
        z.pairs = P("zbl_pairs");
    }
    if (m.cfg.family == RUNE_FAMILY_NEP) {
        m.nep_w0 = P("nep_w0");
        m.nep_b0 = P("nep_b0");
        m.nep_w1 = P("nep_w1");
    } else {
        m.in_w = P("in_w");
        m.in_wT = P("in_wT");
        m.in_b = P("in_b");
        m.emb = P("emb");
        m.res.resize(m.cfg.blocks);
        for (int b = 0; b < m.cfg.blocks; ++b) {
            std::string p = "residual_blocks." + std::to_string(b) + ".";
            m.res[b] = {P(p + "w1"), P(p + "w1T"), P(p + "b1"), P(p + "w2"), P(p + "w2T"),
                        P(p + "b2")};
        }
        m.head_w = P("head_w");
        m.head_b = P("head_b");
        bind_messages(m, P);
    }
    m.host.clear();
    m.finalized = true;
}

// ---------------------------------------------------------------------------
// compute
// ---------------------------------------------------------------------------

// Range check of the atom types.  Writes a copy with every type clamped into
// [0, n_types) -- the kernels after it read the copy, so a bad type never
// indexes past a table -- and flags any type outside the range: a block
// that meets one stores 1 into the flag word (pinned host memory the host
// cleared before the launch), so no clearing launch or copy is needed.
__global__ void __launch_bounds__(1024) k_check_types(int n, const int32_t *types, int n_types,
                                                      int32_t *safe, int32_t *flag) {
    int bad = 0;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int t = types[i];
        const bool out = t < 0 || t >= n_types;
        safe[i] = out ? 0 : t;
        bad |= out;
    }
    bad = __syncthreads_or(bad);
    if (threadIdx.x == 0 && bad) *flag = 1;
}

// Largest atom count checked by one block of k_check_types.
constexpr int kTypeCheckOneBlock = 8192;

static Records records_of(const rune_nlist *nl) {
    Records r;
    r.n_atoms = int(nl->n_atoms);
    r.ptr = nl->ptr.as<int32_t>();
    r.view = nl->view.as<int32_t>();
    r.nbr = nl->nbr.as<int32_t>();
    r.vec = nl->vec.as<float4>();
    r.tptr = nl->tptr.as<int32_t>();
    r.tidx = nl->tidx.as<int32_t>();
    r.tctr = nl->tctr.as<int32_t>();
    r.ctr = nl->ctr.as<int32_t>();
    r.sptr = nl->sptr.as<int32_t>();
    r.n_structures = nl->n_structures;
    r.order = nl->has_order ? nl->order.as<int32_t>() : nullptr;
    r.max_struct_atoms = 0;
    for (size_t b = 0; b + 1 < nl->h_struct_ptr.size(); ++b)
        r.max_struct_atoms = std::max(r.max_struct_atoms,
                                      int(nl->h_struct_ptr[b + 1] - nl->h_struct_ptr[b]));
    return r;
}

// One evaluation.  The workspace is the handle's growing device buffer, or,
// when `fixed` is given, that caller-owned range of `fixed_bytes` bytes (too
// small a range is an argument error, raised before any launch).
static void compute(ModelImpl &m, const rune_nlist *nl, const int32_t *types, int want_f,
                    int want_w, float *d_energies, float *d_energy, float *d_forces,
                    float *d_virial, float *d_atom_virial, hipStream_t s,
                    char *fixed = nullptr, size_t fixed_bytes = 0) {
    RUNE_REQUIRE(m.finalized, RUNE_ERR_STATE, "model handle is not finalized");
    RUNE_REQUIRE(nl, RUNE_ERR_ARGUMENT, "null neighbour list");
    if (!nl->from_padded) {
        RUNE_REQUIRE(nl->rc_radial == m.cfg.rc_radial && nl->rc_angular == m.cfg.rc_angular,
                     RUNE_ERR_STATE, "neighbour list was built with other cutoffs");
    }
    const int N = int(nl->n_atoms);
    const int64_t E = nl->n_records;
    const bool grad = want_f || want_w;
    Records r = records_of(nl);
    nl->order_wanted = m.cfg.family == RUNE_FAMILY_MOBIUS && m.cfg.message_layers > 0;
    const DescTables &d = m.desc;
    const int ldq = (m.Q + 3) & ~3;
    const int nmom = d.na * d.nlm;
    // ---- workspace plan ----
    Arena ar;
    size_t o_types = ar.add(4 * size_t(N));
    size_t o_q = ar.add(4 * size_t(N) * ldq);
    size_t o_dq = ar.add(4 * size_t(N) * ldq);
    size_t o_s = ar.add(4 * size_t(N) * nmom);
    size_t o_e = ar.add(4 * size_t(N));
    size_t o_g = ar.add(16 * size_t(std::max<int64_t>(E, 1)));
    size_t o_av = ar.add(4 * size_t(N) * 9);
    size_t o_f = ar.add(4 * size_t(N) * 3);
    LocalPlan lp = plan_local(m, ar, N);
    MessagePlan mp = plan_messages(m, ar, N, E);
    const size_t o_sums = ar.add(sizeof(double) * std::max<size_t>(1, structure_sum_scratch(r)));
    char *base = fixed;
    if (fixed) {
        if (ar.total > fixed_bytes) {
            std::ostringstream os;
            os << "this evaluation needs " << ar.total << " bytes of workspace; the static "
               << "scratch holds " << fixed_bytes << " (use rune_model_compute)";
            throw Error(RUNE_ERR_ARGUMENT, os.str());
        }
    } else {
        m.work.reserve(ar.total);
        base = m.work.as<char>();
    }
    double *sums = reinterpret_cast<double *>(base + o_sums);
    float *q = reinterpret_cast<float *>(base + o_q);
    float *dq = reinterpret_cast<float *>(base + o_dq);
    float *mom = reinterpret_cast<float *>(base + o_s);
    float *energies = d_energies ? d_energies : reinterpret_cast<float *>(base + o_e);
    float4 *g = reinterpret_cast<float4 *>(base + o_g);
    float *atom_virial = d_atom_virial ? d_atom_virial : reinterpret_cast<float *>(base + o_av);
    float *forces = d_forces ? d_forces : reinterpret_cast<float *>(base + o_f);
    lp.bind(base);
    mp.bind(base);
    // ---- type validation: the flag travels to pinned host memory behind the
    // check kernel and is read once everything else is enqueued, so the
    // host never waits on an idle device; the kernels read the clamped copy
    if (N > 0) {
        int32_t *safe = reinterpret_cast<int32_t *>(base + o_types);
        // a check left in flight by a call that failed part-way must end
        // before the word is cleared
        if (m.type_pending) RUNE_HIP_CHECK(hipEventSynchronize(m.type_event));
        *static_cast<volatile int32_t *>(m.type_flag_host) = 0;
        const int blocks = N <= kTypeCheckOneBlock ? 1 : std::min(ceil_div(N, 1024), 1024);
        hipLaunchKernelGGL(k_check_types, dim3(blocks), dim3(1024), 0, s, N, types, m.cfg.n_types,
                           safe, m.type_flag_host);
        RUNE_HIP_CHECK(hipGetLastError());
        RUNE_HIP_CHECK(hipEventRecord(m.type_event, s));
        m.type_pending = true;
        types = safe;
    }
    if (N == 0) {
        // no atoms: every structure's energy and virial is zero (the sums
        // over empty ranges read nothing)
        structure_sums(r, energies, d_energy, atom_virial, want_w ? d_virial : nullptr, nullptr,
                       s);
        return;
    }
    hipEvent_t *ev = nullptr;
    if (m.timing == 1 && !fixed) {
        if (m.events.empty()) {
            m.events.resize(size_t(kTimingRing) * (RUNE_N_PHASES + 1));
            for (auto &e : m.events) RUNE_HIP_CHECK(hipEventCreate(&e));
        }
        ev = m.events.data() + size_t(m.timed_calls % kTimingRing) * (RUNE_N_PHASES + 1);
        ++m.timed_calls;
    }
    auto mark = [&](int k) {
        if (ev) RUNE_HIP_CHECK(hipEventRecord(ev[k], s));
    };
    // ---- forward ----
    // the message blocks' record-only work runs on the side stream beside the
    // descriptor and the local network; the launch stream waits for it before
    // the blocks (and, whatever happens in between, before compute returns)
    struct SideJoin {
        ModelImpl &m;
        hipStream_t s;
        bool armed = false;
        hipError_t join() {
            if (!armed) return hipSuccess;
            armed = false;
            hipError_t e = hipEventRecord(m.join_ev, m.side);
            return e == hipSuccess ? hipStreamWaitEvent(s, m.join_ev, 0) : e;
        }
        ~SideJoin() { (void)join(); }
    } side_join{m, s};
    if (m.cfg.family == RUNE_FAMILY_MOBIUS) {
        side_join.armed = true;
        side_join.armed = messages_records_ahead(m, mp, r, types, s);
    }
    mark(0);
    descriptor_forward(d, r, E, types, q, ldq, mom, s);
    mark(1);
    const float4 *g_direct = nullptr;
    const float *dmom = nullptr;
    if (m.cfg.family == RUNE_FAMILY_NEP) {
        mark(2);
        mark(3);
        nep_mlp(N, m.Q, m.cfg.nep_hidden, q, ldq, types, m.nep_w0, m.nep_b0, m.nep_w1,
                m.nep_bias, energies, dq, grad ? 1 : 0, s);
        mark(4);
        mark(5);
        mark(6);
    } else {
        float *h = local_forward(m, lp, N, q, ldq, types, s);
        mark(2);
        RUNE_HIP_CHECK(side_join.join());
        h = messages_forward(m, mp, lp, r, types, mom, h, s, grad);
        mark(3);
        float *dh = grad ? lp.dh_a : nullptr;
        readout(N, m.cfg.hidden_dim, h, m.cfg.hidden_dim, types, m.head_w, m.head_b,
                float(m.cfg.norm_eps), energies, dh, m.cfg.hidden_dim, s);
        mark(4);
        if (grad) {
            // the message blocks leave work that feeds only the descriptor
            // reverse on the side stream; joined after the local network
            side_join.armed = m.side != nullptr;
            dh = messages_backward(m, mp, lp, r, types, mom, dh, s);
            mark(5);
            local_backward(m, lp, N, dh, dq, ldq, s);
            RUNE_HIP_CHECK(side_join.join());
            g_direct = mp.g_direct_used ? mp.g_direct : nullptr;
            dmom = mp.dmom_used ? mp.dmom : nullptr;
        } else {
            mark(5);
        }
        mark(6);
    }
    descriptor_reverse(d, m.zbl, r, E, types, dq, ldq, mom, dmom, g_direct, energies, g,
                       grad ? 1 : 0, s);
    mark(7);
    if (grad) forces_and_virial(r, g, forces, atom_virial, s);
    structure_sums(r, energies, d_energy, atom_virial, grad && want_w ? d_virial : nullptr, sums,
                   s);
    mark(8);
    // the type verdict (on a bad type the outputs written above are unspecified)
    RUNE_HIP_CHECK(hipEventSynchronize(m.type_event));
    m.type_pending = false;
    RUNE_REQUIRE(*static_cast<volatile int32_t *>(m.type_flag_host) == 0, RUNE_ERR_TYPE,
                 "atom type outside [0, n_types)");
}

ModelImpl::~ModelImpl() {
    if (side) (void)hipStreamSynchronize(side);
    if (side) (void)hipStreamDestroy(side);
    if (fork_ev) (void)hipEventDestroy(fork_ev);
    if (join_ev) (void)hipEventDestroy(join_ev);
    if (type_event) (void)hipEventDestroy(type_event);
    if (type_flag_host) (void)hipHostFree(type_flag_host);
    for (auto &e : events) (void)hipEventDestroy(e);
    for (auto &e : span_ev) (void)hipEventDestroy(e);
}

int ModelImpl::span_begin(int group, hipStream_t s) {
    if (timing == 0 || span_n >= kMaxSpans) return -1;
    while (span_ev.size() < 2 * (span_n + 1)) {
        hipEvent_t e;
        RUNE_HIP_CHECK(hipEventCreate(&e));
        span_ev.push_back(e);
    }
    if (span_grp.size() < span_n + 1) span_grp.resize(span_n + 1);
    span_grp[span_n] = group;
    RUNE_HIP_CHECK(hipEventRecord(span_ev[2 * span_n], s));
    return int(span_n++);
}

void ModelImpl::span_end(int k, hipStream_t s) {
    if (k >= 0) (void)hipEventRecord(span_ev[2 * size_t(k) + 1], s);
}

// ---- local (descriptor network) part ----

LocalPlan plan_local(ModelImpl &m, Arena &ar, int N) {
    LocalPlan p;
    if (m.cfg.family == RUNE_FAMILY_NEP) return p;
    const int H = m.cfg.hidden_dim, F = m.cfg.ffn_dim, nb = m.cfg.blocks;
    p.o_h = ar.add(4 * size_t(N) * H * (nb + 1));
    p.o_r = ar.add(4 * size_t(N) * std::max(nb, 1));
    p.o_u = ar.add(4 * size_t(N) * F * std::max(nb, 1));
    p.o_a = ar.add(4 * size_t(N) * F);
    p.o_dha = ar.add(4 * size_t(N) * H);
    p.o_dhb = ar.add(4 * size_t(N) * H);
    p.o_dz = ar.add(4 * size_t(N) * H);
    p.N = N;
    p.H = H;
    p.F = F;
    return p;
}

void LocalPlan::bind(char *base) {
    if (!N) return;
    h = reinterpret_cast<float *>(base + o_h);
    r = reinterpret_cast<float *>(base + o_r);
    u = reinterpret_cast<float *>(base + o_u);
    a = reinterpret_cast<float *>(base + o_a);
    dh_a = reinterpret_cast<float *>(base + o_dha);
    dh_b = reinterpret_cast<float *>(base + o_dhb);
    dz = reinterpret_cast<float *>(base + o_dz);
}

float *local_forward(ModelImpl &m, LocalPlan &p, int N, const float *q, int ldq,
                     const int32_t *types, hipStream_t s) {
    const int H = p.H, F = p.F, nb = m.cfg.blocks, act = m.cfg.activation;
    Epilogue e0;
    e0.bias = m.in_b;
    e0.emb = m.emb;
    e0.types = types;
    e0.ld_emb = H;
    gemm(N, H, m.Q, q, ldq, m.in_w, m.Q, p.h, H, e0, s);
    for (int b = 0; b < nb; ++b) {
        float *hb = p.h + size_t(b) * N * H;
        float *hn = p.h + size_t(b + 1) * N * H;
        float *rb = p.r + size_t(b) * N;
        float *ub = p.u + size_t(b) * N * F;
        Epilogue e1;
        e1.rms_out = rb;   // RMSNorm of hb, formed by the GEMM from the rows it reads
        e1.rms_eps = float(m.cfg.norm_eps);
        e1.bias = m.res[b].b1;
        e1.pre = ub;
        e1.ldp = F;
        e1.act = act;
        gemm(N, F, H, hb, H, m.res[b].w1, H, p.a, F, e1, s);
        Epilogue e2;
        e2.bias = m.res[b].b2;
        e2.residual = hb;
        e2.ldr = H;
        gemm(N, H, F, p.a, F, m.res[b].w2, F, hn, H, e2, s);
    }
    return p.h + size_t(nb) * N * H;
}

void local_backward(ModelImpl &m, LocalPlan &p, int N, float *dh, float *dq, int ldq,
                    hipStream_t s) {
    const int H = p.H, F = p.F, nb = m.cfg.blocks, act = m.cfg.activation;
    float *cur = dh;
    float *other = (dh == p.dh_a) ? p.dh_b : p.dh_a;
    for (int b = nb - 1; b >= 0; --b) {
        float *hb = p.h + size_t(b) * N * H;
        float *rb = p.r + size_t(b) * N;
        float *ub = p.u + size_t(b) * N * F;
        Epilogue e1;
        e1.dact_from = ub;
        e1.ldu = F;
        e1.dact = act;
        gemm(N, F, H, cur, H, m.res[b].w2T, H, p.a, F, e1, s);      // du
        Epilogue e2;
        gemm(N, H, F, p.a, F, m.res[b].w1T, F, p.dz, H, e2, s);     // dz
        rms_backward(N, H, hb, H, rb, p.dz, H, cur, H, other, H, s);
        std::swap(cur, other);
    }
    Epilogue e3;
    gemm(N, m.Q, H, cur, H, m.in_wT, H, dq, ldq, e3, s);
}

}  // namespace rune

using namespace rune;

extern "C" const char *rune_last_error(void) { return g_last_error_ptr(); }

extern "C" const char *rune_version(void) { return "rune_hip 0.1.0 (gfx950)"; }

extern "C" int rune_model_create(const rune_model_config *config, rune_model **out) {
    return guarded([&] {
        RUNE_REQUIRE(config && out, RUNE_ERR_ARGUMENT, "null argument");
        const rune_model_config &c = *config;
        RUNE_REQUIRE(c.n_types >= 1, RUNE_ERR_ARGUMENT, "n_types must be positive");
        RUNE_REQUIRE(c.n_desc_radial >= 1 && c.k_radial >= 1 && c.n_desc_angular >= 1 &&
                         c.k_angular >= 1, RUNE_ERR_ARGUMENT,
                     "descriptor channel counts and basis sizes must be positive");
        RUNE_REQUIRE(c.l_max >= 1 && c.l_max <= kMaxL, RUNE_ERR_ARGUMENT, "l_max outside [1, 8]");
        {
            // the descriptor kernels for wide models keep per-lane rows of
            // the basis and channel values in LDS (one 64-lane wave per atom)
            int num_L = c.l_max;
            for (int k = 0; k < 6; ++k) num_L += c.has_q[k] ? 1 : 0;
            const size_t nlm = size_t(c.l_max) * (c.l_max + 2), na = c.n_desc_angular;
            const size_t kmax = std::max(c.k_radial, c.k_angular);
            const size_t Q = c.n_desc_radial + na * num_L;
            const size_t lds = 4 * std::max(64 * (kmax + 1 + na + 1 + nlm + 1) + na * nlm,
                                            Q + 2 * na * nlm + 128 * (kmax + 1) + 128 * (na + 1));
            RUNE_REQUIRE(lds <= 160 * 1024, RUNE_ERR_ARGUMENT,
                         "descriptor too wide for one 64-lane wave per atom (n_max / basis_size "
                         "need more than 160 KB of LDS)");
        }
        RUNE_REQUIRE(c.rc_radial > 0 && c.rc_angular > 0, RUNE_ERR_ARGUMENT, "bad cutoffs");
        if ((c.has_q[0] || c.has_q[2]) && c.l_max < 2)
            throw Error(RUNE_ERR_ARGUMENT, "q222 / q112 require l_max >= 2");
        if ((c.has_q[3] || c.has_q[4]) && c.l_max < 3)
            throw Error(RUNE_ERR_ARGUMENT, "q_123 and q_233 require l_max >= 3.");
        if (c.has_q[5] && c.l_max < 4)
            throw Error(RUNE_ERR_ARGUMENT, "q_134 requires l_max >= 4.");
        auto *m = new rune_model();
        m->cfg = c;
        m->cfg.elements = nullptr;
        if (c.elements)
            for (int t = 0; t < c.n_types; ++t) m->elements.push_back(str(c.elements[t]));
        if (c.family == RUNE_FAMILY_NEP && int(m->elements.size()) != c.n_types) {
            delete m;
            throw Error(RUNE_ERR_ARGUMENT, "NEP models need the element symbols");
        }
        int num_L = c.l_max;
        for (int k = 0; k < 6; ++k) num_L += c.has_q[k] ? 1 : 0;
        m->Q = c.n_desc_radial + c.n_desc_angular * num_L;
        DescTables &d = m->desc;
        d.n_types = c.n_types;
        d.nr = c.n_desc_radial;
        d.kr = c.k_radial;
        d.na = c.n_desc_angular;
        d.ka = c.k_angular;
        d.l_max = c.l_max;
        d.nlm = c.l_max * (c.l_max + 2);
        d.num_L = num_L;
        d.Q = m->Q;
        for (int k = 0; k < 6; ++k) d.has_q[k] = c.has_q[k] ? 1 : 0;
        d.rc_r = float(c.rc_radial);
        d.rc_a = float(c.rc_angular);
        ZblTables &z = m->zbl;
        z.mode = c.zbl_mode;
        z.n_types = c.n_types;
        z.rc_inner = float(c.zbl_rc_inner);
        z.rc_outer = float(c.zbl_rc_outer);
        z.on_angular = c.family == RUNE_FAMILY_NEP ? 1 : 0;
        try {
            validate_messages(*m);
            define_expected(*m);
        } catch (...) {
            delete m;
            throw;
        }
        *out = m;
    });
}

extern "C" void rune_model_destroy(rune_model *model) { delete model; }

extern "C" int rune_model_set_tensor(rune_model *model, const char *name, const float *h_data,
                                     int64_t n_elements) {
    return guarded([&] {
        RUNE_REQUIRE(model && name, RUNE_ERR_ARGUMENT, "null argument");
        RUNE_REQUIRE(!model->finalized, RUNE_ERR_STATE, "model is already finalized");
        auto it = model->expected.find(name);
        RUNE_REQUIRE(it != model->expected.end(), RUNE_ERR_ARGUMENT,
                     std::string("unexpected state_dict key ") + name);
        if (it->second != n_elements) {
            std::ostringstream os;
            os << "size mismatch for " << name << ": expected " << it->second << " values, got "
               << n_elements;
            throw Error(RUNE_ERR_ARGUMENT, os.str());
        }
        RUNE_REQUIRE(h_data || n_elements == 0, RUNE_ERR_ARGUMENT, "null data");
        model->host[name].assign(h_data, h_data + n_elements);
    });
}

extern "C" int rune_model_finalize(rune_model *model) {
    return guarded([&] {
        RUNE_REQUIRE(model, RUNE_ERR_ARGUMENT, "null model");
        finalize(*model);
    });
}

extern "C" int rune_model_compute(rune_model *model, const rune_nlist *nl, const int32_t *d_types,
                                  int32_t compute_forces, int32_t compute_virial,
                                  float *d_energies, float *d_energy, float *d_forces,
                                  float *d_virial, float *d_atom_virial, void *stream) {
    return guarded([&] {
        RUNE_REQUIRE(model, RUNE_ERR_ARGUMENT, "null model");
        compute(*model, nl, d_types, compute_forces, compute_virial, d_energies, d_energy,
                d_forces, d_virial, d_atom_virial, as_stream(stream));
    });
}

// ---------------------------------------------------------------------------
// rune_model_compute_static: the evaluation with its workspace in a static
// device array instead of the handle's allocation.
// ---------------------------------------------------------------------------

// 64 MiB per GPU the library runs on, held until the process ends.  Host code
// must not use the array's name as a device address: each device's copy is
// found once with hipGetSymbolAddress and kept in g_scratch_addr.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

namespace rune {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
char *g_scratch_addr[kMaxDevices] = {};

// Device address of the current device's scratch copy (resolved on the first
// call on that device, with that device current).
char *static_scratch() {
    int dev = 0;
    RUNE_HIP_CHECK(hipGetDevice(&dev));
    RUNE_REQUIRE(dev >= 0 && dev < kMaxDevices, RUNE_ERR_STATE, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_addr[dev]) {
        void *addr = nullptr;
        RUNE_HIP_CHECK(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
        RUNE_REQUIRE(addr != nullptr, RUNE_ERR_HIP, "static scratch has no device address");
        g_scratch_addr[dev] = static_cast<char *>(addr);
    }
    return g_scratch_addr[dev];
}
}  // namespace
}  // namespace rune

extern "C" int rune_model_compute_static(rune_model *model, const rune_nlist *nl,
                                         const int32_t *d_types, int32_t compute_forces,
                                         int32_t compute_virial, float *d_energies,
                                         float *d_energy, float *d_forces, float *d_virial,
                                         float *d_atom_virial, void *stream) {
    return guarded([&] {
        RUNE_REQUIRE(model, RUNE_ERR_ARGUMENT, "null model");
        char *ws = static_scratch();
        // no timing events here (creating them is a runtime allocation)
        struct Untimed {
            ModelImpl &m;
            int was;
            explicit Untimed(ModelImpl &x) : m(x), was(x.timing) { m.timing = 0; }
            ~Untimed() { m.timing = was; }
        } untimed(*model);
        compute(*model, nl, d_types, compute_forces, compute_virial, d_energies, d_energy,
                d_forces, d_virial, d_atom_virial, as_stream(stream), ws, kStaticScratchBytes);
    });
}

extern "C" int64_t rune_model_static_scratch_bytes(void) { return int64_t(kStaticScratchBytes); }

namespace rune {
namespace {
// GPUMD's per-atom arrays (rune/mobius/src/force.cu:47-84): potential[n],
// forces as three atom arrays, the virial as nine atom arrays in the order
// xx, yy, zz, xy, xz, yz, yx, zx, zy of -r (x) g, i.e. component (a, b) is
// this library's atom virial W[b][a].  Added in fp64, one thread per atom.
__global__ void k_gpumd_accumulate(int n, const float *e, const float *f, const float *w,
                                   double *pot, double *force, double *vir) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (pot) pot[i] += double(e[i]);
    if (force)
        for (int d = 0; d < 3; ++d) force[size_t(d) * n + i] += double(f[3 * size_t(i) + d]);
    if (vir) {
        const int a[9] = {0, 1, 2, 0, 0, 1, 1, 2, 2}, b[9] = {0, 1, 2, 1, 2, 2, 0, 0, 1};
        for (int k = 0; k < 9; ++k)
            vir[size_t(k) * n + i] += double(w[9 * size_t(i) + 3 * b[k] + a[k]]);
    }
}
}  // namespace
}  // namespace rune

extern "C" int rune_model_compute_gpumd(rune_model *model, const rune_nlist *nl,
                                        const int32_t *d_types, double *d_potential,
                                        double *d_force, double *d_virial, void *stream) {
    return guarded([&] {
        RUNE_REQUIRE(model && nl, RUNE_ERR_ARGUMENT, "null argument");
        const int64_t n = nl->n_atoms;
        hipStream_t s = as_stream(stream);
        model->gpumd_out.reserve(4 * size_t(std::max<int64_t>(n, 1)) * 13);
        float *e = model->gpumd_out.as<float>(), *f = e + n, *w = f + 3 * n;
        compute(*model, nl, d_types, 1, d_virial != nullptr, e, nullptr, f, nullptr,
                d_virial ? w : nullptr, s);
        if (n > 0)
            hipLaunchKernelGGL(k_gpumd_accumulate, dim3(ceil_div(n, 256)), dim3(256), 0, s,
                               int(n), e, f, w, d_potential, d_force, d_virial);
        RUNE_HIP_CHECK(hipGetLastError());
    });
}

namespace rune {
namespace {
// Column extrema of q [n, ldq] (first Q columns), one block per column; NaN
// propagates as in torch.amin / torch.minimum.  accumulate: combine with the
// values already in qmin / qmax.
__device__ inline float nan_min(float a, float b) { return (a < b || a != a) ? a : b; }
__device__ inline float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }

__global__ void __launch_bounds__(256) k_column_extrema(int n, const float *q, int ldq,
                                                        float *qmin, float *qmax, int accumulate) {
    __shared__ float smin[256], smax[256];
    const int col = blockIdx.x, t = threadIdx.x;
    float lo = INFINITY, hi = -INFINITY;
    for (int i = t; i < n; i += 256) {
        const float v = q[size_t(i) * ldq + col];
        lo = nan_min(v, lo);
        hi = nan_max(v, hi);
    }
    smin[t] = lo;
    smax[t] = hi;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) {
            smin[t] = nan_min(smin[t + w], smin[t]);
            smax[t] = nan_max(smax[t + w], smax[t]);
        }
        __syncthreads();
    }
    if (t == 0) {
        qmin[col] = accumulate ? nan_min(smin[0], qmin[col]) : smin[0];
        qmax[col] = accumulate ? nan_max(smax[0], qmax[col]) : smax[0];
    }
}
}  // namespace
}  // namespace rune

extern "C" int rune_model_descriptor_extrema(rune_model *model, const rune_nlist *nl,
                                             const int32_t *d_types, float *d_q_min,
                                             float *d_q_max, int32_t accumulate, void *stream) {
    return guarded([&] {
        RUNE_REQUIRE(model && nl && d_q_min && d_q_max, RUNE_ERR_ARGUMENT, "null argument");
        ModelImpl &m = *model;
        RUNE_REQUIRE(m.finalized, RUNE_ERR_STATE, "model handle is not finalized");
        if (!nl->from_padded)
            RUNE_REQUIRE(nl->rc_radial == m.cfg.rc_radial && nl->rc_angular == m.cfg.rc_angular,
                         RUNE_ERR_STATE, "neighbour list was built with other cutoffs");
        hipStream_t s = as_stream(stream);
        const int N = int(nl->n_atoms);
        const DescTables &d = m.desc;
        const int ldq = (m.Q + 3) & ~3;
        Arena ar;
        const size_t o_flag = ar.add(16);
        const size_t o_types = ar.add(4 * size_t(std::max(N, 1)));
        const size_t o_q = ar.add(4 * size_t(std::max(N, 1)) * ldq);
        const size_t o_s = ar.add(4 * size_t(std::max(N, 1)) * d.na * d.nlm);
        m.work.reserve(ar.total);
        char *base = m.work.as<char>();
        int32_t *flag = reinterpret_cast<int32_t *>(base + o_flag);
        RUNE_HIP_CHECK(hipMemsetAsync(flag, 0, 16, s));
        if (N > 0)
            hipLaunchKernelGGL(k_check_types, dim3(std::min(ceil_div(N, 1024), 1024)), dim3(1024),
                               0, s, N, d_types, m.cfg.n_types,
                               reinterpret_cast<int32_t *>(base + o_types), flag);
        int32_t hflag = 0;
        RUNE_HIP_CHECK(hipMemcpyAsync(&hflag, flag, 4, hipMemcpyDeviceToHost, s));
        RUNE_HIP_CHECK(hipStreamSynchronize(s));
        RUNE_REQUIRE(hflag == 0, RUNE_ERR_TYPE, "atom type outside [0, n_types)");
        float *q = reinterpret_cast<float *>(base + o_q);
        if (N > 0)
            descriptor_forward(d, records_of(nl), nl->n_records, d_types, q, ldq,
                               reinterpret_cast<float *>(base + o_s), s);
        hipLaunchKernelGGL(k_column_extrema, dim3(m.Q), dim3(256), 0, s, N, q, ldq, d_q_min,
                           d_q_max, int(accumulate != 0));
        RUNE_HIP_CHECK(hipGetLastError());
    });
}

extern "C" int32_t rune_model_input_dim(const rune_model *model) { return model ? model->Q : 0; }

extern "C" int rune_model_supports_heat_current(const rune_model *model) {
    return model && (model->cfg.family == RUNE_FAMILY_NEP || model->cfg.message_layers == 0) ? 1
                                                                                            : 0;
}

extern "C" int64_t rune_model_workspace_bytes(const rune_model *model) {
    return model ? int64_t(model->work.bytes) : 0;
}

extern "C" int rune_model_timing(rune_model *model, int32_t enable) {
    return guarded([&] {
        RUNE_REQUIRE(model, RUNE_ERR_ARGUMENT, "null model");
        RUNE_REQUIRE(enable >= 0 && enable <= 2, RUNE_ERR_ARGUMENT, "timing mode is 0, 1 or 2");
        model->timing = enable;
        model->timed_calls = 0;
        model->span_n = 0;
    });
}

extern "C" int rune_model_timing_groups(rune_model *model, double *ms, int64_t *launches) {
    return guarded([&] {
        RUNE_REQUIRE(model && ms, RUNE_ERR_ARGUMENT, "null argument");
        for (int k = 0; k < RUNE_N_GROUPS; ++k) {
            ms[k] = 0.0;
            if (launches) launches[k] = 0;
        }
        for (size_t k = 0; k < model->span_n; ++k) {
            RUNE_HIP_CHECK(hipEventSynchronize(model->span_ev[2 * k + 1]));
            float t = 0.0f;
            RUNE_HIP_CHECK(hipEventElapsedTime(&t, model->span_ev[2 * k],
                                               model->span_ev[2 * k + 1]));
            const int g = model->span_grp[k];
            ms[g] += t;
            if (launches) ++launches[g];
        }
    });
}

extern "C" int rune_model_timing_read(rune_model *model, double *ms, int64_t *calls) {
    return guarded([&] {
        RUNE_REQUIRE(model && ms, RUNE_ERR_ARGUMENT, "null argument");
        for (int k = 0; k < RUNE_N_PHASES; ++k) ms[k] = 0.0;
        int64_t n = std::min<int64_t>(model->timed_calls, kTimingRing);
        for (int64_t c = 0; c < n; ++c) {
            hipEvent_t *ev = model->events.data() + size_t(c) * (RUNE_N_PHASES + 1);
            RUNE_HIP_CHECK(hipEventSynchronize(ev[RUNE_N_PHASES]));
            for (int k = 0; k < RUNE_N_PHASES; ++k) {
                float t = 0.0f;
                RUNE_HIP_CHECK(hipEventElapsedTime(&t, ev[k], ev[k + 1]));
                ms[k] += t;
            }
        }
        if (calls) *calls = n;
    });
}
