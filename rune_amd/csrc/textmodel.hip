// Native readers of the two text artifacts, so a C/C++ caller needs no
// PyTorch pickle:
//   mobius1 (rune/mobius/export.py:120-146), read and validated as the GPUMD
//     evaluator does (rune/mobius/src/mobius.cu:26-151): elements, schema 1,
//     ints, reals, tensors (the state_dict plus derived `desc.*` tables), END;
//   nep4 / nep4_zbl (rune/nep/model.py:284-489): header lines, then the
//     per-element ANN, the shared bias, the two c-tables (file order n, k, t1,
//     t2), the q scaler and the flexible ZBL rows.
// Both end in rune_model_create / rune_model_set_tensor / rune_model_finalize
// with the state_dict names the PyTorch loaders would pass.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdlib>
#include <fstream>
#include <map>
#include <set>
#include <sstream>

#include "model.hpp"
#include "text_tables.hpp"

namespace rune {
namespace {

struct TextTensor {
    std::vector<int64_t> dims;
    std::vector<double> values;
};

[[noreturn]] void bad(const std::string &msg) { throw Error(RUNE_ERR_ARGUMENT, msg); }

void require_text(bool ok, const std::string &msg) {
    if (!ok) bad(msg);
}

void expect_word(std::istream &in, const char *word) {
    std::string actual;
    require_text(bool(in >> actual) && actual == word,
                 std::string("expected '") + word + "' in model file");
}

// Reads one real with the C library (handles nan / inf spellings and hex).
bool read_real(std::istream &in, double &v) {
    std::string t;
    if (!(in >> t)) return false;
    char *end = nullptr;
    v = std::strtod(t.c_str(), &end);
    return end && *end == '\0' && end != t.c_str();
}

bool read_int(std::istream &in, int64_t &v) {
    std::string t;
    if (!(in >> t)) return false;
    char *end = nullptr;
    v = std::strtoll(t.c_str(), &end, 10);
    return end && *end == '\0' && end != t.c_str();
}

void check_call(int rc) {
    if (rc != RUNE_OK) throw Error(rc, rune_last_error());
}

// Order L of angular component k (components of order L at L*L-1 .. L*L+2L-1).
int order_of_component(int k) {
    int L = 1;
    while ((L + 1) * (L + 1) - 1 <= k) ++L;
    return L;
}

// Which higher-order invariants a mobius1 file carries, from its sparse
// invariant table: channels past l_max appear in the order q222, q1111, q112,
// q123, q233, q134 (enabled ones only); each is recognised by the orders of
// its first term's components (2,2,2 / 1,1,1,1 / 1,1,2 / 1,2,3 / 2,3,3 / 1,3,4).
void invariant_flags(const TextTensor &terms, const TextTensor &offsets, int l_max, int num_L,
                     int32_t *has_q) {
    for (int k = 0; k < 6; ++k) has_q[k] = 0;
    require_text(terms.dims.size() == 2 && terms.dims[1] == 7 &&
                     int64_t(offsets.values.size()) == num_L + 1,
                 "invalid descriptor polynomial tables");
    const std::vector<std::vector<int>> sig = {
        {2, 2, 2}, {1, 1, 1, 1}, {1, 1, 2}, {1, 2, 3}, {2, 3, 3}, {1, 3, 4}};
    int last = -1;
    for (int ch = l_max; ch < num_L; ++ch) {
        const int64_t row = int64_t(offsets.values[ch]);
        require_text(row >= 0 && row < terms.dims[0], "invalid descriptor polynomial tables");
        const double *r = terms.values.data() + row * 7;
        const int degree = int(r[2]);
        require_text(degree >= 1 && degree <= 4, "invalid descriptor polynomial tables");
        std::vector<int> orders;
        for (int d = 0; d < degree; ++d) orders.push_back(order_of_component(int(r[3 + d])));
        std::sort(orders.begin(), orders.end());
        int kind = -1;
        for (int k = 0; k < 6; ++k)
            if (orders == sig[k]) kind = k;
        require_text(kind > last, "unrecognised invariant table of the model file");
        has_q[kind] = 1;
        last = kind;
    }
}

rune_model *load_mobius(std::istream &in) {
    int64_t count = 0, schema = 0;
    require_text(read_int(in, count) && count > 0 && count <= 118, "invalid element count");
    std::vector<std::string> elements(count);
    for (auto &e : elements) require_text(bool(in >> e), "missing element");
    require_text(std::set<std::string>(elements.begin(), elements.end()).size() ==
                     elements.size(),
                 "duplicate elements");
    expect_word(in, "schema");
    require_text(read_int(in, schema) && schema == 1, "unsupported native schema");
    std::map<std::string, int64_t> ints;
    std::map<std::string, double> reals;
    std::map<std::string, TextTensor> tensors;
    std::vector<std::string> tensor_order;
    expect_word(in, "ints");
    require_text(read_int(in, count) && count > 0 && count < 1000,
                 "invalid integer metadata count");
    for (int64_t k = 0; k < count; ++k) {
        std::string key;
        int64_t v = 0;
        require_text(bool(in >> key) && read_int(in, v), "invalid integer metadata");
        require_text(ints.emplace(key, v).second, "duplicate integer metadata");
    }
    expect_word(in, "reals");
    require_text(read_int(in, count) && count > 0 && count < 1000, "invalid real metadata count");
    for (int64_t k = 0; k < count; ++k) {
        std::string key;
        double v = 0;
        require_text(bool(in >> key) && read_real(in, v) && std::isfinite(v),
                     "invalid real metadata");
        require_text(reals.emplace(key, v).second, "duplicate real metadata");
    }
    expect_word(in, "tensors");
    require_text(read_int(in, count) && count > 0 && count < 100000, "invalid tensor count");
    for (int64_t k = 0; k < count; ++k) {
        std::string key;
        int64_t rank = 0;
        require_text(bool(in >> key) && read_int(in, rank) && rank >= 0 && rank <= 8,
                     "invalid tensor rank");
        TextTensor t;
        int64_t size = 1;
        for (int64_t a = 0; a < rank; ++a) {
            int64_t d = 0;
            require_text(read_int(in, d) && d >= 0, "invalid tensor dimension");
            require_text(d == 0 || size <= (int64_t(1) << 31) / d, "tensor is too large");
            size *= d;
            t.dims.push_back(d);
        }
        t.values.resize(size_t(size));
        for (double &v : t.values)
            require_text(read_real(in, v) && std::isfinite(v),
                         "missing or nonfinite tensor values");
        require_text(tensors.emplace(key, std::move(t)).second, "duplicate tensor name");
        tensor_order.push_back(key);
    }
    expect_word(in, "END");
    std::string trailing;
    require_text(!(in >> trailing), "unexpected data after END");
    auto I = [&](const char *key) -> int64_t {
        auto it = ints.find(key);
        require_text(it != ints.end(), std::string("missing integer metadata ") + key);
        return it->second;
    };
    auto R = [&](const char *key) -> double {
        auto it = reals.find(key);
        require_text(it != reals.end(), std::string("missing real metadata ") + key);
        return it->second;
    };
    require_text(I("n_types") == int64_t(elements.size()), "element count mismatch");
    for (const char *key : {"n_desc_radial", "n_desc_angular", "k_max_radial", "k_max_angular",
                            "num_L", "input_dim", "hidden_dim", "ffn_dim", "message_dim",
                            "pair_dim", "message_groups", "message_basis_size"})
        require_text(I(key) > 0, std::string("invalid ") + key);
    require_text(I("message_layers") >= 0 && I("blocks") >= 0, "negative layer count");
    require_text(I("activation") >= 0 && I("activation") <= 2, "unsupported activation");
    require_text(I("message_mode") == 0 || I("message_mode") == 1, "unsupported message mode");
    require_text(I("l_max") >= 1 && I("l_max") <= 8, "unsupported angular order");
    require_text(!I("message_layers") || I("hidden_dim") % I("message_groups") == 0,
                 "invalid message groups");
    require_text(R("rcut_radial") > 0 && R("rcut_angular") > 0 && R("message_cutoff") > 0 &&
                     R("norm_eps") > 0,
                 "cutoffs and normalization epsilon must be positive");
    require_text(R("message_cutoff") <= R("rcut_radial"), "message cutoff exceeds radial cutoff");
    require_text(I("max_neighbors_radial") > 0 && I("max_neighbors_angular") > 0 &&
                     I("vector_channels") >= 0,
                 "invalid neighbor/channel capacity");
    require_text(I("input_dim") == I("n_desc_radial") + I("n_desc_angular") * I("num_L"),
                 "descriptor dimension mismatch");
    const bool eq = I("message_mode") == 1;
    require_text(!eq || (I("equivariant_channels") > 0 && I("equivariant_l_max") >= 1 &&
                         I("equivariant_l_max") <= I("l_max") && I("message_layers") > 0),
                 "invalid equivariant dimensions");
    auto need = [&](const char *name) -> const TextTensor & {
        auto it = tensors.find(name);
        require_text(it != tensors.end(), std::string("missing tensor '") + name + "'");
        return it->second;
    };
    rune_model_config c{};
    c.family = RUNE_FAMILY_MOBIUS;
    c.n_types = int32_t(elements.size());
    c.n_desc_radial = int32_t(I("n_desc_radial"));
    c.k_radial = int32_t(I("k_max_radial"));
    c.n_desc_angular = int32_t(I("n_desc_angular"));
    c.k_angular = int32_t(I("k_max_angular"));
    c.l_max = int32_t(I("l_max"));
    invariant_flags(need("desc.invariant_terms"), need("desc.invariant_offsets"), c.l_max,
                    int(I("num_L")), c.has_q);
    c.rc_radial = R("rcut_radial");
    c.rc_angular = R("rcut_angular");
    c.hidden_dim = int32_t(I("hidden_dim"));
    c.ffn_dim = int32_t(I("ffn_dim"));
    c.blocks = int32_t(I("blocks"));
    c.activation = int32_t(I("activation"));
    c.message_layers = int32_t(I("message_layers"));
    c.message_mode = eq ? RUNE_MESSAGE_EQUIVARIANT : RUNE_MESSAGE_SCALAR;
    c.message_dim = int32_t(I("message_dim"));
    c.pair_dim = int32_t(I("pair_dim"));
    c.message_groups = int32_t(I("message_groups"));
    c.vector_channels = int32_t(I("vector_channels"));
    c.message_basis_size = int32_t(I("message_basis_size"));
    c.equivariant_channels = int32_t(I("equivariant_channels"));
    c.equivariant_l_max = int32_t(I("equivariant_l_max"));
    c.message_cutoff = R("message_cutoff");
    c.norm_eps = R("norm_eps");
    if (I("zbl_enabled")) {
        c.zbl_mode = I("zbl_flexible") ? RUNE_ZBL_FLEXIBLE : RUNE_ZBL_UNIVERSAL;
        c.zbl_rc_inner = R("zbl_rc_inner");
        c.zbl_rc_outer = R("zbl_rc_outer");
    } else {
        c.zbl_mode = RUNE_ZBL_NONE;
    }
    std::vector<const char *> names;
    for (const auto &e : elements) names.push_back(e.c_str());
    c.elements = names.data();
    rune_model *m = nullptr;
    check_call(rune_model_create(&c, &m));
    try {
        for (const auto &key : tensor_order) {
            if (key.rfind("desc.", 0) == 0) continue;   // derived tables of the native format
            const TextTensor &t = tensors[key];
            std::vector<float> f(t.values.begin(), t.values.end());
            check_call(rune_model_set_tensor(m, key.c_str(), f.data(), int64_t(f.size())));
        }
        check_call(rune_model_finalize(m));
    } catch (...) {
        rune_model_destroy(m);
        throw;
    }
    m->max_radial = int(I("max_neighbors_radial"));
    m->max_angular = int(I("max_neighbors_angular"));
    return m;
}

std::vector<std::string> split(const std::string &line) {
    std::istringstream is(line);
    std::vector<std::string> out;
    std::string t;
    while (is >> t) out.push_back(t);
    return out;
}

double to_real(const std::string &t, const char *what) {
    char *end = nullptr;
    const double v = std::strtod(t.c_str(), &end);
    require_text(end && *end == '\0' && end != t.c_str(), std::string("Invalid nep.txt: ") + what);
    return v;
}

int64_t to_int(const std::string &t, const char *what) {
    char *end = nullptr;
    const long long v = std::strtoll(t.c_str(), &end, 10);
    require_text(end && *end == '\0' && end != t.c_str(), std::string("Invalid nep.txt: ") + what);
    return v;
}

rune_model *load_nep(const std::vector<std::string> &lines) {
    size_t idx = 0;
    std::vector<std::string> tok = split(lines[idx++]);
    std::string head = tok[0];
    std::transform(head.begin(), head.end(), head.begin(), ::tolower);
    require_text(head.rfind("nep", 0) == 0 && head.size() > 3 && std::isdigit(head[3]),
                 "Invalid nep.txt: first line should start with nep4 or nep5.");
    size_t p = 3;
    while (p < head.size() && std::isdigit(head[p])) ++p;
    require_text(std::atoi(head.substr(3, p - 3).c_str()) == 4,
                 "Only nep4 is supported by the RUNE loader.");
    bool has_zbl = false;
    if (p < head.size()) {
        require_text(head[p] == '_', "Invalid nep.txt: first line should start with nep4 or nep5.");
        std::istringstream rest(head.substr(p + 1));
        std::string part;
        while (std::getline(rest, part, '_')) has_zbl = has_zbl || part == "zbl";
    }
    require_text(tok.size() >= 2, "Invalid nep.txt: element count mismatch.");
    const int T = int(to_int(tok[1], "element count"));
    std::vector<std::string> elements(tok.begin() + 2, tok.end());
    require_text(T >= 1 && int(elements.size()) == T, "Invalid nep.txt: element count mismatch.");
    for (const auto &e : elements) {
        bool known = false;
        for (int z = 1; z < int(sizeof(text_tables::kSymbols) / sizeof(char *)); ++z)
            known = known || e == text_tables::kSymbols[z];
        require_text(known, "Invalid nep.txt: unknown element " + e);
    }
    auto next_line = [&]() -> std::vector<std::string> {
        require_text(idx < lines.size(), "Invalid nep.txt: unexpected end of file.");
        return split(lines[idx++]);
    };
    double zbl_inner = 0, zbl_outer = 0;
    bool zbl_flexible = false;
    if (has_zbl) {
        tok = next_line();
        require_text(tok[0] == "zbl" && (tok.size() == 3 || tok.size() == 4),
                     "Invalid nep.txt: zbl line not found after nep4_zbl header.");
        require_text(tok.size() == 3, "Typewise ZBL cutoffs are not supported in RUNE.");
        zbl_inner = to_real(tok[1], "zbl line");
        zbl_outer = to_real(tok[2], "zbl line");
        zbl_flexible = zbl_inner == 0.0 && zbl_outer == 0.0;
    }
    tok = next_line();
    require_text(tok[0] == "cutoff", "Invalid nep.txt: cutoff line not found.");
    double rc_r = 0, rc_a = 0;
    int64_t mn_r = 0, mn_a = 0;
    if (tok.size() == 5) {
        rc_r = to_real(tok[1], "cutoff line");
        rc_a = to_real(tok[2], "cutoff line");
        mn_r = to_int(tok[3], "cutoff line");
        mn_a = to_int(tok[4], "cutoff line");
    } else {
        require_text(int(tok.size()) == 2 * T + 3, "Invalid nep.txt: cutoff line length mismatch.");
        std::set<double> rr, ra;
        for (int t = 0; t < T; ++t) {
            rr.insert(to_real(tok[1 + 2 * t], "cutoff line"));
            ra.insert(to_real(tok[2 + 2 * t], "cutoff line"));
        }
        require_text(rr.size() == 1 && ra.size() == 1, "Per-type cutoffs are not supported in RUNE.");
        rc_r = *rr.begin();
        rc_a = *ra.begin();
        mn_r = to_int(tok[tok.size() - 2], "cutoff line");
        mn_a = to_int(tok[tok.size() - 1], "cutoff line");
    }
    auto keyed = [&](const char *key) {
        std::vector<std::string> t = next_line();
        require_text(!t.empty() && t[0] == key, std::string("Invalid nep.txt: ") + key +
                                                    " line not found.");
        return t;
    };
    tok = keyed("n_max");
    require_text(tok.size() >= 3, "Invalid nep.txt: n_max line not found.");
    const int n_r = int(to_int(tok[1], "n_max")), n_a = int(to_int(tok[2], "n_max"));
    tok = keyed("basis_size");
    require_text(tok.size() >= 3, "Invalid nep.txt: basis_size line not found.");
    const int b_r = int(to_int(tok[1], "basis_size")), b_a = int(to_int(tok[2], "basis_size"));
    tok = keyed("l_max");
    std::vector<int> lv;
    for (size_t k = 1; k < tok.size(); ++k) lv.push_back(int(to_int(tok[k], "l_max")));
    require_text(lv.size() >= 1 && lv.size() <= 7,
                 "Invalid nep.txt: l_max should contain 1 to 7 values.");
    const int defaults[6] = {1, 0, 0, 0, 0, 0};
    for (size_t k = lv.size(); k < 7; ++k) lv.push_back(defaults[k - 1]);
    tok = next_line();
    require_text(tok[0] == "ANN" && tok.size() == 3, "Invalid nep.txt: expected ANN width 0.");
    const int hidden = int(to_int(tok[1], "ANN"));
    require_text(hidden >= 1 && hidden <= 200, "Invalid nep.txt: ANN width must be in [1, 200].");
    require_text(to_int(tok[2], "ANN") == 0,
                 "RUNE only supports single-hidden-layer NEP text models (ANN width 0).");
    rune_model_config c{};
    c.family = RUNE_FAMILY_NEP;
    c.n_types = T;
    c.n_desc_radial = n_r + 1;
    c.k_radial = b_r + 1;
    c.n_desc_angular = n_a + 1;
    c.k_angular = b_a + 1;
    c.l_max = lv[0];
    for (int k = 0; k < 6; ++k) c.has_q[k] = lv[1 + k] > 0 ? 1 : 0;
    c.rc_radial = rc_r;
    c.rc_angular = rc_a;
    c.nep_hidden = hidden;
    c.zbl_mode = !has_zbl ? RUNE_ZBL_NONE : zbl_flexible ? RUNE_ZBL_FLEXIBLE : RUNE_ZBL_UNIVERSAL;
    c.zbl_rc_inner = zbl_inner;
    c.zbl_rc_outer = zbl_outer;
    require_text(!has_zbl || zbl_flexible || (0.0 <= zbl_inner && zbl_inner < zbl_outer),
                 "Universal ZBL requires 0 <= rc_inner < rc_outer.");
    int num_L = c.l_max;
    for (int k = 0; k < 6; ++k) num_L += c.has_q[k];
    const int dim = c.n_desc_radial + c.n_desc_angular * num_L;
    // all remaining values, each rounded to fp32 as the PyTorch reader does
    std::vector<float> values;
    for (; idx < lines.size(); ++idx)
        for (const auto &t : split(lines[idx])) values.push_back(float(to_real(t, "parameter")));
    size_t pos = 0;
    auto take = [&](size_t n) {
        require_text(pos + n <= values.size(), "Invalid nep.txt: not enough parameters.");
        std::vector<float> out(values.begin() + pos, values.begin() + pos + n);
        pos += n;
        return out;
    };
    std::vector<std::pair<std::string, std::vector<float>>> sd;
    for (const auto &e : elements) {
        const std::string p0 = "element_mlps." + e + ".";
        sd.emplace_back(p0 + "0.weight", take(size_t(hidden) * dim));
        std::vector<float> b = take(hidden);
        for (float &v : b) v = -v;
        sd.emplace_back(p0 + "0.bias", b);
        sd.emplace_back(p0 + "2.weight", take(hidden));
    }
    sd.emplace_back("shared_bias", take(1));
    const char *table_names[2] = {"descriptor.radial.c_table", "descriptor.angular.c_table"};
    const int nds[2] = {n_r + 1, n_a + 1}, kks[2] = {b_r + 1, b_a + 1};
    for (int w = 0; w < 2; ++w) {
        const int nd = nds[w], kk = kks[w];
        const std::vector<float> flat = take(size_t(nd) * kk * T * T);
        std::vector<float> tab(flat.size());
        for (int n = 0; n < nd; ++n)
            for (int k = 0; k < kk; ++k)
                for (int t1 = 0; t1 < T; ++t1)
                    for (int t2 = 0; t2 < T; ++t2)
                        tab[((size_t(t1) * T + t2) * nd + n) * kk + k] =
                            flat[((size_t(n) * kk + k) * T + t1) * T + t2];
        sd.emplace_back(table_names[w], tab);
    }
    sd.emplace_back("q_scaler", take(dim));
    auto constants = [&](const char *name, const double *v, size_t n) {
        sd.emplace_back(name, std::vector<float>(v, v + n));
    };
    constants("descriptor.angular.C3B", text_tables::kC3B, 80);
    constants("descriptor.angular.C4B", text_tables::kC4B, 5);
    constants("descriptor.angular.C5B", text_tables::kC5B, 3);
    constants("descriptor.angular.C4B2", text_tables::kC4B2, 5);
    const double *zs[8] = {text_tables::kZ1, text_tables::kZ2, text_tables::kZ3, text_tables::kZ4,
                           text_tables::kZ5, text_tables::kZ6, text_tables::kZ7, text_tables::kZ8};
    for (int L = 1; L <= 8; ++L)
        sd.emplace_back("descriptor.angular.Z" + std::to_string(L),
                        std::vector<float>(zs[L - 1], zs[L - 1] + (L + 1) * (L + 1)));
    if (has_zbl) {
        std::vector<float> z;
        for (const auto &e : elements)
            for (int n = 1; n < int(sizeof(text_tables::kSymbols) / sizeof(char *)); ++n)
                if (e == text_tables::kSymbols[n]) z.push_back(float(n));
        sd.emplace_back("zbl.atomic_numbers", z);
        constants("zbl.universal_coefficients", text_tables::kUniversalZbl, 8);
        std::vector<float> rows;
        if (zbl_flexible) {
            rows.assign(values.begin() + pos, values.end());
            pos = values.size();
            require_text(rows.size() == size_t(T) * (T + 1) / 2 * 10,
                         "Flexible ZBL expects " + std::to_string(T * (T + 1) / 2) +
                             " pair rows.");
            for (float v : rows)
                require_text(std::isfinite(v), "Flexible ZBL parameters must all be finite.");
            for (size_t r = 0; r < rows.size(); r += 10)
                require_text(rows[r] >= 0.0f && rows[r] < rows[r + 1],
                             "Each flexible ZBL pair must satisfy 0 <= rc_inner < rc_outer.");
        }
        sd.emplace_back("zbl.pair_parameters", rows);
    }
    std::vector<const char *> names;
    for (const auto &e : elements) names.push_back(e.c_str());
    c.elements = names.data();
    rune_model *m = nullptr;
    check_call(rune_model_create(&c, &m));
    try {
        for (const auto &kv : sd)
            check_call(rune_model_set_tensor(m, kv.first.c_str(), kv.second.data(),
                                             int64_t(kv.second.size())));
        check_call(rune_model_finalize(m));
    } catch (...) {
        rune_model_destroy(m);
        throw;
    }
    m->max_radial = int(mn_r);
    m->max_angular = int(mn_a);
    return m;
}

}  // namespace
}  // namespace rune

using namespace rune;

extern "C" int rune_model_load(const char *path, rune_model **out) {
    return guarded([&] {
        RUNE_REQUIRE(path && out, RUNE_ERR_ARGUMENT, "null argument");
        *out = nullptr;
        std::ifstream in(path);
        RUNE_REQUIRE(bool(in), RUNE_ERR_ARGUMENT, std::string("cannot open ") + path);
        std::string first;
        RUNE_REQUIRE(bool(in >> first), RUNE_ERR_ARGUMENT, "empty model file");
        if (first == "mobius1") {
            *out = load_mobius(in);
            return;
        }
        in.clear();
        in.seekg(0);
        std::vector<std::string> lines;
        std::string line;
        while (std::getline(in, line))
            if (line.find_first_not_of(" \t\r") != std::string::npos) lines.push_back(line);
        *out = load_nep(lines);
    });
}

extern "C" int rune_model_limits(const rune_model *model, double *rc_radial, double *rc_angular,
                                 int32_t *max_radial, int32_t *max_angular) {
    return guarded([&] {
        RUNE_REQUIRE(model, RUNE_ERR_ARGUMENT, "null model");
        if (rc_radial) *rc_radial = model->cfg.rc_radial;
        if (rc_angular) *rc_angular = model->cfg.rc_angular;
        if (max_radial) *max_radial = model->max_radial;
        if (max_angular) *max_angular = model->max_angular;
    });
}

extern "C" const char *rune_model_element(const rune_model *model, int32_t type) {
    if (!model || type < 0 || type >= int32_t(model->elements.size())) return "";
    return model->elements[type].c_str();
}
