// Schema-specialised kernels: source generation and hipRTC compilation.
//
// For a derivative schema the sigmoid composition (replacing the reference's
// hand-written d1..d6 / d1p..d6p, cuda/derivative_kernels_v4.cu:12-745) is
// emitted as straight-line register code: every multiset-partition term with
// its integer coefficient, every product of stack rows computed once (products
// are built from shared prefixes), every adjoint pair (cuda/cpde_engine.cuh:476-498)
// unrolled.  The generated functions are prepended to the layer-fused kernel
// templates (fused.hip.in) and the module is compiled for the device's
// architecture with hipRTC -- the way the reference compiles its expression
// costs with NVRTC (cuda/expression_program.hpp:96-131).
//
// Compiled code objects are cached on disk, keyed by a hash of the source and
// the options: $CPDE_JIT_CACHE, else <library directory>/../jit_cache.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>

#include "common.hpp"

namespace cpde {

extern const char* const kFusedSource;  // fused.hip.in, embedded at build time

namespace {

float word_float(int w) {
    float f;
    std::memcpy(&f, &w, sizeof f);
    return f;
}

std::string flit(float f) {
    char buf[48];
    std::snprintf(buf, sizeof buf, "%.9gf", double(f));
    std::string s(buf);
    if (s.find_first_of(".eEn") == std::string::npos) s.insert(s.size() - 1, ".0");
    return s;
}

struct Products {
    std::ostringstream& out;
    std::map<std::vector<int>, std::string> names;
    std::string get(const std::vector<int>& rows) {
        if (rows.size() == 1) return "z[" + std::to_string(rows[0]) + "]";
        auto it = names.find(rows);
        if (it != names.end()) return it->second;
        std::vector<int> prefix(rows.begin(), rows.end() - 1);
        const std::string a = get(prefix);
        std::string name = "p";
        for (int r : rows) name += "_" + std::to_string(r);
        out << "    const float " << name << " = " << a << " * z[" << rows.back() << "];\n";
        names[rows] = name;
        return name;
    }
};

// The sigma derivatives from q = 1/(1+e^z) (cuda/derivative_kernels_v4.cu:462-468).
void emit_sigma(std::ostringstream& o, int highest) {
    o << "    const float q = 1.0f / (1.0f + expf(z[0]));\n";
    o << "    const float s1 = q * (1.0f - q);\n";
    if (highest >= 2) o << "    const float s2 = -s1 * (1.0f - 2.0f * q);\n";
    if (highest >= 3) o << "    const float s3 = s1 * (1.0f - 6.0f * s1);\n";
    if (highest >= 4) o << "    const float s4 = s2 * (1.0f - 12.0f * s1);\n";
    if (highest >= 5) o << "    const float s5 = s1 - (5.0f * s2) * (6.0f * s2);\n";
    if (highest >= 6) o << "    const float s6 = s2 + 5.0f * (s4 - s2) * (1.0f - 6.0f * s1);\n";
    if (highest >= 7)
        o << "    const float s7 = (5.0f * s1) * (0.2f - (8.4f * s1) * (3.0f - 4.0f * (5.0f * s1 + 5.0f * s3)));\n";
}

// sum_m s_{m+shift} M_m for row r, M_m = sum_terms c * prod(block rows).  With
// `prime`, also sum_m s_{m+1} M_m (the row of the jet of sigma') into *prime.
std::string emit_partition_sum(std::ostringstream& o, Products& P, const Tables& t, int r, int shift,
                               const std::string& name, std::string* prime = nullptr) {
    int pos = t.fwd_offset[r];
    const int k = t.words[pos++];
    std::string acc, pacc;
    for (int m = 1; m <= k; ++m) {
        const int count = t.words[pos++];
        std::string M = "0.0f";
        for (int q = 0; q < count; ++q) {
            const float c = word_float(t.words[pos]);
            const unsigned w0 = unsigned(t.words[pos + 1]), w1 = unsigned(t.words[pos + 2]);
            pos += 3;
            std::vector<int> rows;
            for (int b = 0; b < m; ++b) rows.push_back(int(((b < 4 ? w0 >> (8 * b) : w1 >> (8 * (b - 4)))) & 255u));
            const std::string prod = P.get(rows);
            if (q == 0 && c == 1.0f)
                M = prod;
            else if (q == 0)
                M = flit(c) + " * " + prod;
            else
                M = "fmaf(" + flit(c) + ", " + prod + ", " + M + ")";
            if (q + 1 < count && M.size() > 200) {  // keep expressions short
                const std::string tmp = name + "_m" + std::to_string(m) + "_" + std::to_string(q);
                o << "    const float " << tmp << " = " << M << ";\n";
                M = tmp;
            }
        }
        if (prime) {  // M is used twice
            const std::string tmp = name + "_M" + std::to_string(m);
            o << "    const float " << tmp << " = " << M << ";\n";
            M = tmp;
        }
        const std::string s = "s" + std::to_string(m + shift);
        acc = m == 1 ? s + " * " + M : "fmaf(" + s + ", " + M + ", " + acc + ")";
        const std::string tmp = name + "_a" + std::to_string(m);
        o << "    const float " << tmp << " = " << acc << ";\n";
        acc = tmp;
        if (prime) {
            const std::string sp = "s" + std::to_string(m + shift + 1);
            pacc = m == 1 ? sp + " * " + M : "fmaf(" + sp + ", " + M + ", " + pacc + ")";
            const std::string ptmp = name + "_u" + std::to_string(m);
            o << "    const float " << ptmp << " = " << pacc << ";\n";
            pacc = ptmp;
        }
    }
    if (prime) *prime = pacc;
    return acc;
}

}  // namespace

namespace {

int forward_terms(const Tables& t, int r) {
    if (r == 0) return 1;
    int pos = t.fwd_offset[r];
    const int k = t.words[pos++];
    int terms = 0;
    for (int m = 1; m <= k; ++m) {
        const int count = t.words[pos++];
        terms += count;
        pos += 3 * count;
    }
    return terms;
}

// Rows split into G groups of balanced cost (greedy, largest first).
std::vector<int> row_groups(int rows, int G, const std::vector<int>& cost) {
    std::vector<int> order(rows), group(rows, 0);
    for (int r = 0; r < rows; ++r) order[r] = r;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cost[a] > cost[b]; });
    std::vector<long> load(G, 0);
    for (int r : order) {
        const int g = int(std::min_element(load.begin(), load.end()) - load.begin());
        group[r] = g;
        load[g] += cost[r];
    }
    return group;
}

// compose_forward rows where owned[r]; the others of y are left untouched.
void emit_forward(std::ostringstream& o, const Tables& t, const std::string& name, const std::vector<char>& owned) {
    o << "__device__ __forceinline__ void " << name << "(const float* __restrict__ z, float* __restrict__ y) {\n";
    emit_sigma(o, std::max(1, t.max_order));
    if (owned[0]) o << "    y[0] = 1.0f / (1.0f + expf(-z[0]));\n";
    Products P{o, {}};
    for (int r = 1; r < t.rows; ++r) {
        if (!owned[r]) continue;
        const std::string v = emit_partition_sum(o, P, t, r, 0, "f" + std::to_string(r));
        o << "    y[" << r << "] = " << v << ";\n";
    }
    o << "}\n";
}

// The same rows of y and of u, the jet of sigma'(z) (u[0] = sigma'(z0)): the
// partition sums M_m of a row serve both, y = sum s_m M_m and u = sum s_{m+1} M_m.
void emit_forward_prime(std::ostringstream& o, const Tables& t, const std::string& name,
                        const std::vector<char>& owned) {
    o << "__device__ __forceinline__ void " << name
      << "(const float* __restrict__ z, float* __restrict__ y, float* __restrict__ u) {\n";
    emit_sigma(o, t.max_order + 1);
    if (owned[0]) o << "    y[0] = 1.0f / (1.0f + expf(-z[0]));\n    u[0] = s1;\n";
    Products P{o, {}};
    for (int r = 1; r < t.rows; ++r) {
        if (!owned[r]) continue;
        std::string prime;
        const std::string v = emit_partition_sum(o, P, t, r, 0, "f" + std::to_string(r), &prime);
        o << "    y[" << r << "] = " << v << ";\n    u[" << r << "] = " << prime << ";\n";
    }
    o << "}\n";
}

// compose_adjoint outputs gz[i] where owned[i]; the others are left untouched.
void emit_adjoint(std::ostringstream& o, const Tables& t, const std::string& name, const std::vector<char>& owned) {
    o << "__device__ __forceinline__ void " << name << "(const float* __restrict__ z, const float* __restrict__ gy,"
         " float* __restrict__ gz) {\n";
    emit_sigma(o, t.max_order + 1);
    std::vector<char> needed(t.rows, 0);
    for (int i = 0; i < t.rows; ++i) {
        if (!owned[i]) continue;
        int pos = t.pair_offset[i];
        const int count = t.words[pos++];
        for (int q = 0; q < count; ++q, pos += 3) needed[t.words[pos + 1]] = 1;
    }
    Products P{o, {}};
    for (int r = 1; r < t.rows; ++r) {
        if (!needed[r]) continue;
        const std::string v = emit_partition_sum(o, P, t, r, 1, "d" + std::to_string(r));
        o << "    const float D" << r << " = " << v << ";\n";
    }
    for (int i = 0; i < t.rows; ++i) {
        if (!owned[i]) continue;
        int pos = t.pair_offset[i];
        const int count = t.words[pos++];
        o << "    { float acc = s1 * gy[" << i << "];\n";
        for (int q = 0; q < count; ++q, pos += 3) {
            const int j = t.words[pos], dn = t.words[pos + 1];
            require(dn > 0, "adjoint pair refers to the value row");
            const float c = word_float(t.words[pos + 2]);
            o << "      acc = acc + (" << flit(c) << " * gy[" << j << "]) * D" << dn << ";\n";
        }
        o << "      gz[" << i << "] = acc; }\n";
    }
    o << "}\n";
}

// The adjoint from the jet of sigma' kept by the forward:
// gz_i = u_0 gy_i + sum over pairs C(alpha_j, alpha_i) gy_j u_(alpha_j - alpha_i)
// (back_step, cuda/derivative_kernels_v4.cu:349-380, with DPlus = u).
void emit_adjoint_prime(std::ostringstream& o, const Tables& t, const std::string& name,
                        const std::vector<char>& owned) {
    o << "__device__ __forceinline__ void " << name << "(const float* __restrict__ u, const float* __restrict__ gy,"
         " float* __restrict__ gz) {\n";
    for (int i = 0; i < t.rows; ++i) {
        if (!owned[i]) continue;
        int pos = t.pair_offset[i];
        const int count = t.words[pos++];
        o << "    { float acc = u[0] * gy[" << i << "];\n";
        for (int q = 0; q < count; ++q, pos += 3) {
            const int j = t.words[pos], dn = t.words[pos + 1];
            require(dn > 0, "adjoint pair refers to the value row");
            const float c = word_float(t.words[pos + 2]);
            if (c == 1.0f)
                o << "      acc = fmaf(gy[" << j << "], u[" << dn << "], acc);\n";
            else
                o << "      acc = fmaf(" << flit(c) << " * gy[" << j << "], u[" << dn << "], acc);\n";
        }
        o << "      gz[" << i << "] = acc; }\n";
    }
    o << "}\n";
}

// ---- Taylor-scaled rows ------------------------------------------------------
// A scaled stack holds row alpha as d^alpha f / alpha!, the Taylor coefficient.
// Linear steps commute with the scaling, Leibniz products lose their binomials,
// and sigma' = sigma (1 - sigma) closes a recurrence over the orders:
//   y_a = (1/a_i) sum_{b <= a - e_i} u_b (a_i - b_i) z_{a-b}   (y' = sigma'(z) z' along x_i)
//   u_a = y_a (1 - 2 y_0) - sum_{0 < c < a} y_c y_{a-c}        (u = y - y^2)
// with u the jet of sigma'(z), and the adjoint of y = sigma(z) is
//   gz_b = sum_{a >= b} u_{a-b} gy_a.
// For 2 variables through order 6 the recurrence takes 307 operations where the
// partition sums take 706, and the adjoint 210 fused multiply-adds where the
// binomial pairs take 335 operations.

struct Jet {
    int V = 0, R = 0;
    std::vector<std::vector<int>> alpha;  // multi-index of each row
    std::map<std::vector<int>, int> row;  // row of each multi-index
    explicit Jet(const Tables& t) : V(t.variables), R(t.rows), alpha(t.rows) {
        for (int r = 0; r < R; ++r) {
            alpha[r].assign(t.table.begin() + r * (V + 1) + 1, t.table.begin() + (r + 1) * (V + 1));
            row[alpha[r]] = r;
        }
    }
    int find(const std::vector<int>& a) const {
        const auto it = row.find(a);
        return it == row.end() ? -1 : it->second;
    }
    static bool below(const std::vector<int>& b, const std::vector<int>& a) {  // b <= a componentwise
        for (size_t j = 0; j < a.size(); ++j)
            if (b[j] > a[j]) return false;
        return true;
    }
    static std::vector<int> minus(std::vector<int> a, const std::vector<int>& b) {
        for (size_t j = 0; j < a.size(); ++j) a[j] -= b[j];
        return a;
    }
    int order(int r) const {
        int s = 0;
        for (int c : alpha[r]) s += c;
        return s;
    }
    int mirror(int r) const {  // the row with variables 0 and 1 swapped, -1 if absent
        if (V < 2) return -1;
        std::vector<int> a = alpha[r];
        std::swap(a[0], a[1]);
        return find(a);
    }
};

// y[0] = sigma(z0), u[0] = sigma'(z0) = sigma(z0) sigma(-z0) and c0 = 1 - 2 sigma(z0)
// from e^{-|z0|}, which cannot overflow; no cancellation at either tail.
void emit_scaled_sigmoid(std::ostringstream& o) {
    o << "    const float E = __expf(-fabsf(z[0]));\n"
         "    const float sp = __builtin_amdgcn_rcpf(1.0f + E);\n"  // sigma(|z0|)
         "    const float sn = E * sp;\n"                           // sigma(-|z0|)
         "    const bool pos = z[0] >= 0.0f;\n"
         "    y[0] = pos ? sp : sn;\n"
         "    u[0] = sp * sn;\n"
         "    const float c0 = pos ? sn - sp : sp - sn;\n";
}

// Scaled y and u of every row from scaled z.  `mirror`: the lane computes the
// rows with alpha_0 >= alpha_1 of its own jet, and at the end of each order
// takes the others from its partner lane (the adjacent lane, which runs the
// same code on the jet with variables 0 and 1 swapped, so its row mirror(b)
// is this lane's row b).
void emit_scaled_forward(std::ostringstream& o, const Tables& t, const std::string& name, bool mirror) {
    const Jet J(t);
    o << "__device__ __forceinline__ void " << name
      << "(const float* __restrict__ z, float* __restrict__ y, float* __restrict__ u) {\n";
    emit_scaled_sigmoid(o);
    std::map<std::pair<int, int>, std::string> directional;  // (i, r) -> delta_i * z[r]
    auto zdir = [&](int i, int r) -> std::string {
        const int d = J.alpha[r][i];
        if (d == 1) return "z[" + std::to_string(r) + "]";
        auto it = directional.find({i, r});
        if (it != directional.end()) return it->second;
        const std::string nm = "zd" + std::to_string(i) + "_" + std::to_string(r);
        o << "    const float " << nm << " = " << flit(float(d)) << " * z[" << r << "];\n";
        directional[{i, r}] = nm;
        return nm;
    };
    for (int r = 1; r < J.R; ++r) {
        const std::vector<int>& a = J.alpha[r];
        if (!mirror || a[0] >= a[1]) {
            int i = -1;  // the direction with the fewest terms: smallest positive count
            for (int j = 0; j < J.V; ++j)
                if (a[j] > 0 && (i < 0 || a[j] < a[i])) i = j;
            std::vector<int> am = a;
            --am[i];
            std::string acc;
            int terms = 0;
            for (int b = 0; b < J.R; ++b) {
                if (!Jet::below(J.alpha[b], am)) continue;
                const int d = J.find(Jet::minus(a, J.alpha[b]));
                require(d > 0, "scaled composition: schema is not closed");
                const std::string zt = zdir(i, d);
                const std::string ub = "u[" + std::to_string(b) + "]";
                acc = acc.empty() ? ub + " * " + zt : "fmaf(" + ub + ", " + zt + ", " + acc + ")";
                if (++terms % 8 == 0) {  // keep expressions short
                    const std::string tmp = "f" + std::to_string(r) + "_" + std::to_string(terms);
                    o << "    const float " << tmp << " = " << acc << ";\n";
                    acc = tmp;
                }
            }
            if (a[i] >= 2) acc = "(" + acc + ") * " + flit(1.0f / float(a[i]));
            o << "    y[" << r << "] = " << acc << ";\n";
            o << "    { float s = y[" << r << "] * c0;\n";
            std::string pairs;
            for (int c = 1; c < J.R; ++c) {
                if (c == r || !Jet::below(J.alpha[c], a)) continue;
                const int h = J.find(Jet::minus(a, J.alpha[c]));
                if (h < c) continue;  // each unordered pair once
                if (h == c)
                    o << "      s = fmaf(-y[" << c << "], y[" << c << "], s);\n";
                else {
                    const std::string prod = "y[" + std::to_string(c) + "], y[" + std::to_string(h) + "]";
                    pairs = pairs.empty() ? "y[" + std::to_string(c) + "] * y[" + std::to_string(h) + "]"
                                          : "fmaf(" + prod + ", " + pairs + ")";
                }
            }
            if (!pairs.empty()) o << "      s = fmaf(-2.0f, " << pairs << ", s);\n";
            o << "      u[" << r << "] = s; }\n";
        }
        if (mirror && (r + 1 == J.R || J.order(r + 1) != J.order(r)))
            for (int b = 1; b <= r; ++b) {
                if (J.order(b) != J.order(r) || J.alpha[b][0] >= J.alpha[b][1]) continue;
                const int m = J.mirror(b);
                require(m >= 0, "mirror split: schema is not symmetric");
                o << "    y[" << b << "] = partner(y[" << m << "]);\n    u[" << b << "] = partner(u[" << m << "]);\n";
            }
    }
    o << "}\n";
}

// Scaled adjoint rows gz_b = sum_{a >= b} u_{a-b} gy_a where owned[b].
void emit_scaled_adjoint(std::ostringstream& o, const Tables& t, const std::string& name,
                         const std::vector<char>& owned) {
    const Jet J(t);
    o << "__device__ __forceinline__ void " << name << "(const float* __restrict__ u, const float* __restrict__ gy,"
         " float* __restrict__ gz) {\n";
    for (int b = 0; b < J.R; ++b) {
        if (!owned[b]) continue;
        o << "    { float acc = u[0] * gy[" << b << "];\n";
        for (int a = b + 1; a < J.R; ++a) {
            if (!Jet::below(J.alpha[b], J.alpha[a])) continue;
            const int d = J.find(Jet::minus(J.alpha[a], J.alpha[b]));
            require(d > 0, "scaled adjoint: schema is not closed");
            o << "      acc = fmaf(u[" << d << "], gy[" << a << "], acc);\n";
        }
        o << "      gz[" << b << "] = acc; }\n";
    }
    o << "}\n";
}

int scaled_adjoint_terms(const Jet& J, int b) {
    int n = 1;
    for (int a = b + 1; a < J.R; ++a) n += Jet::below(J.alpha[b], J.alpha[a]);
    return n;
}

}  // namespace

bool mirror_symmetric(const Tables& t) {
    const Jet J(t);
    if (J.V < 2) return false;
    for (int r = 0; r < J.R; ++r)
        if (J.mirror(r) < 0) return false;
    return true;
}

// compose_forward / compose_adjoint (from z) and compose_forward_prime /
// compose_adjoint_prime (keeping and contracting the jet of sigma') for all
// rows, and for each G in `splits` the G partial versions of the latter,
// compose_forward_G<G>_<g> / compose_adjoint_G<G>_<g>, plus the row-to-group
// tables kForwardGroup<G>[R] / kAdjointGroup<G>[R].
// `scaled`: the _prime functions (and the adjoint's partial versions) work on
// Taylor-scaled rows, the forward splits over two mirror lanes
// (compose_forward_mirror) instead of row groups, and kRowScale[R] = alpha!
// and kRowUnscale[R] = 1/alpha! convert rows.
std::string compose_source(const Tables& t, const std::vector<int>& splits, bool scaled) {
    std::ostringstream o;
    o << "#define CPDE_R " << t.rows << "\n";
    const std::vector<char> all(t.rows, 1);
    emit_forward(o, t, "compose_forward", all);
    emit_adjoint(o, t, "compose_adjoint", all);
    if (scaled) {
        const Jet J(t);
        std::vector<float> fact(t.rows, 1.0f);
        for (int r = 0; r < t.rows; ++r)
            for (int c : J.alpha[r])
                for (int k = 2; k <= c; ++k) fact[r] *= float(k);
        o << "constexpr float kRowScale[" << t.rows << "] = {";
        for (int r = 0; r < t.rows; ++r) o << (r ? ", " : "") << flit(fact[r]);
        o << "};\n__constant__ float kRowScaleTable[" << t.rows << "] = {";
        for (int r = 0; r < t.rows; ++r) o << (r ? ", " : "") << flit(fact[r]);
        o << "};\nconstexpr float kRowUnscale[" << t.rows << "] = {";
        for (int r = 0; r < t.rows; ++r) o << (r ? ", " : "") << flit(1.0f / fact[r]);
        o << "};\n";
        // the partner lane's copy of a value (adjacent lanes 2j, 2j+1: quad_perm [1,0,3,2])
        o << "__device__ __forceinline__ float partner(float v) {\n"
             "    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));\n}\n";
        emit_scaled_forward(o, t, "compose_forward_prime", false);
        if (mirror_symmetric(t)) {
            o << "#define CPDE_MIRROR 1\nconstexpr unsigned char kMirror[" << t.rows << "] = {";
            for (int r = 0; r < t.rows; ++r) o << (r ? ", " : "") << J.mirror(r);
            o << "};\n";
            emit_scaled_forward(o, t, "compose_forward_mirror", true);
        }
        emit_scaled_adjoint(o, t, "compose_adjoint_prime", all);
        std::vector<int> acost(t.rows);
        for (int r = 0; r < t.rows; ++r) acost[r] = scaled_adjoint_terms(J, r);
        for (int G : splits) {
            if (G <= 1) continue;
            const std::vector<int> ag = row_groups(t.rows, G, acost);
            o << "constexpr unsigned char kAdjointGroup" << G << "[" << t.rows << "] = {";
            for (int r = 0; r < t.rows; ++r) o << (r ? ", " : "") << ag[r];
            o << "};\n";
            for (int g = 0; g < G; ++g) {
                std::vector<char> owned(t.rows, 0);
                for (int r = 0; r < t.rows; ++r) owned[r] = ag[r] == g;
                emit_scaled_adjoint(o, t, "compose_adjoint_G" + std::to_string(G) + "_" + std::to_string(g), owned);
            }
        }
        return o.str();
    }
    emit_forward_prime(o, t, "compose_forward_prime", all);
    emit_adjoint_prime(o, t, "compose_adjoint_prime", all);
    std::vector<int> fcost(t.rows), acost(t.rows);
    for (int r = 0; r < t.rows; ++r) {
        fcost[r] = forward_terms(t, r) + 1;
        acost[r] = t.words[t.pair_offset[r]] + 1;
    }
    for (int G : splits) {
        if (G <= 1) continue;
        const std::vector<int> fg = row_groups(t.rows, G, fcost), ag = row_groups(t.rows, G, acost);
        for (int which = 0; which < 2; ++which) {
            const std::vector<int>& grp = which ? ag : fg;
            o << "constexpr unsigned char k" << (which ? "Adjoint" : "Forward") << "Group" << G << "[" << t.rows
              << "] = {";
            for (int r = 0; r < t.rows; ++r) o << (r ? ", " : "") << grp[r];
            o << "};\n";
            for (int g = 0; g < G; ++g) {
                std::vector<char> owned(t.rows, 0);
                for (int r = 0; r < t.rows; ++r) owned[r] = grp[r] == g;
                const std::string name = std::string(which ? "compose_adjoint_G" : "compose_forward_G") +
                                         std::to_string(G) + "_" + std::to_string(g);
                if (which) emit_adjoint_prime(o, t, name, owned);
                else emit_forward_prime(o, t, name, owned);
            }
        }
    }
    return o.str();
}

namespace {

uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

std::string cache_dir() {
    if (const char* env = std::getenv("CPDE_JIT_CACHE")) return env;
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&fnv1a), &info) && info.dli_fname) {
        std::string lib(info.dli_fname);
        const size_t slash = lib.rfind('/');
        if (slash != std::string::npos) return lib.substr(0, slash) + "/../jit_cache";
    }
    return "";
}

bool read_file(const std::string& path, std::vector<char>& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    return !out.empty();
}

void write_file(const std::string& path, const std::vector<char>& data) {
    const std::string tmp = path + ".tmp" + std::to_string(getpid());
    {
        std::ofstream f(tmp, std::ios::binary);
        if (!f) return;
        f.write(data.data(), std::streamsize(data.size()));
        if (!f) return;
    }
    std::rename(tmp.c_str(), path.c_str());
}

std::mutex compile_mutex;

}  // namespace

// Compiles (or fetches from the cache) the code object of `source` for `arch`.
std::vector<char> compile_module(const std::string& source, const std::string& arch, std::string* log) {
    const std::string arch_opt = "--offload-arch=" + arch;
    const char* options[] = {arch_opt.c_str(), "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                             "-packed-fp32-ops"};
    const int noptions = int(sizeof options / sizeof options[0]);
    std::string key_text = source;
    for (auto* opt : options) key_text += std::string("\n") + opt;
    char name[64];
    std::snprintf(name, sizeof name, "cpde_%016llx.co", (unsigned long long)fnv1a(key_text));
    const std::string dir = cache_dir();
    const std::string path = dir.empty() ? "" : dir + "/" + name;
    std::vector<char> code;
    std::lock_guard<std::mutex> lock(compile_mutex);
    if (const char* dump = std::getenv("CPDE_JIT_DUMP")) {  // source of the last module, for inspection
        std::ofstream f(dump);
        f << source;
    }
    if (!path.empty() && read_file(path, code)) return code;
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, source.c_str(), "cpde_fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        throw compile_error("hiprtcCreateProgram failed");
    const hiprtcResult result = hiprtcCompileProgram(prog, noptions, options);
    size_t size = 0;
    hiprtcGetProgramLogSize(prog, &size);
    std::string text(size, '\0');
    if (size) hiprtcGetProgramLog(prog, &text[0]);
    while (!text.empty() && text.back() == '\0') text.pop_back();
    if (log) *log = text;
    if (result != HIPRTC_SUCCESS) {
        hiprtcDestroyProgram(&prog);
        throw compile_error("fused kernel compile failed: " + text.substr(0, 4000));
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    code.resize(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    if (!path.empty()) {
        mkdir(dir.c_str(), 0755);
        write_file(path, code);
    }
    return code;
}

// Most lanes per forward composition: scaled compositions split only over the
// two mirror images of a symmetric schema.
static int forward_split_cap(const Tables& t, const FusedTuning& tuning) {
    if (!tuning.scaled) return tuning.max_split;
    return mirror_symmetric(t) ? std::min(tuning.max_split, 2) : 1;
}

// Whether every hidden layer's forward and adjoint compositions have one lane
// per (point, neuron) column (the row split of fused.hip.in's split_of is 1).
static bool alias_tiles(const Tables& t, const std::vector<int>& neurons, const FusedTuning& tuning) {
    for (size_t l = 1; l + 1 < neurons.size(); ++l) {
        const int lanes = tuning.net_points_per_block * neurons[l], T = tuning.net_threads;
        const int G = lanes * 4 <= T ? 4 : (lanes * 2 <= T ? 2 : 1);
        if (std::min(G, forward_split_cap(t, tuning)) != 1 || std::min(G, tuning.max_split_adjoint) != 1) return false;
    }
    return true;
}

// The network kernels' LDS tiles: the operand tile X and the product tile T,
// which is X itself under CPDE_ALIAS_TILES.
static std::string tile_declarations() {
    return "    __shared__ __attribute__((aligned(16))) float X[kNNC * kS];\n"
           "#ifdef CPDE_ALIAS_TILES\n"
           "    float* const T = X;\n"
           "#else\n"
           "    __shared__ __attribute__((aligned(16))) float T[kNNC * kS];\n"
           "#endif\n";
}

// Tuning macros, the generated compositions and the fused kernels' device code
// for a schema and architecture.
static void emit_prologue(std::ostream& o, const Tables& t, const std::vector<int>& neurons,
                          const FusedTuning& tuning) {
    const int points_per_block = tuning.points_per_block, net_points_per_block = tuning.net_points_per_block;
    const int L = int(neurons.size());
    int widest = 0;
    for (int l = 1; l + 1 < L; ++l) widest = std::max(widest, neurons[l]);
    o << "// generated: cPDE layer-fused kernels\n#define CPDE_POINTS " << points_per_block << "\n";
    o << "#define CPDE_NET_POINTS " << net_points_per_block << "\n";
    o << "#define CPDE_NET_THREADS " << tuning.net_threads << "\n";
    o << "#define CPDE_STRIDE " << ((widest + 7) / 8 * 8 + 4) << "\n";
    // Column tile of the network products: 16 (v_mfma_f32_16x16x4f32) or 32
    // (v_mfma_f32_32x32x2f32), as the tuning chose it; without a choice, 16 when
    // a block holds one point.  16 needs every hidden width a multiple of 16.
    // Measured on 2->128^4->1 at 729 points, epoch kernel: one point per block
    // (orders 5, 6; 21 and 28 rows) 16 is 6 and 2 % faster, and 35 rows pad to
    // 48 columns instead of 64 (3D order 4: 11 %).
    {
        bool hidden16 = true;
        for (int l = 1; l + 1 < L; ++l) hidden16 = hidden16 && neurons[l] % 16 == 0;
        int col_tile = net_points_per_block == 1 ? 16 : 32;
        if (tuning.col_tile == 16 || tuning.col_tile == 32) col_tile = tuning.col_tile;
        if (!hidden16) col_tile = 32;
        o << "#define CPDE_COL_TILE " << col_tile << "\n";
    }
    const int forward_cap = forward_split_cap(t, tuning);
    o << "#define CPDE_MAX_SPLIT " << forward_cap << "\n";
    // One LDS tile instead of two when every composition has whole columns per
    // lane (no split): a lane then reads a column's z rows and writes its y
    // rows in place, and the products wait for every wave's operand reads
    // before they store.  Half the LDS per workgroup.
    if (tuning.alias && alias_tiles(t, neurons, tuning)) o << "#define CPDE_ALIAS_TILES 1\n";
    o << "#define CPDE_MAX_SPLIT_ADJOINT " << tuning.max_split_adjoint << "\n";
    if (tuning.scaled) o << "#define CPDE_SCALED 1\n";
    if (tuning.inkernel_wgrad) o << "#define CPDE_INKERNEL_WGRAD 1\n";
    if (tuning.b_pairs) o << "#define CPDE_B_PAIRS 1\n";
    if (tuning.stamps) o << "#define CPDE_STAMPS 1\n";
    if (tuning.tier_prio) o << "#define CPDE_TIER_PRIO " << tuning.tier_prio << "\n#define CPDE_TIER_CUS " << tuning.tier_cus << "\n";
    // row splits of the compositions used by the network-fused kernels (scaled
    // forward compositions split over mirror lanes instead)
    std::vector<int> splits;
    for (int l = 1; l + 1 < L; ++l) {
        const int lanes = net_points_per_block * neurons[l], T = tuning.net_threads;
        const int G = lanes * 4 <= T ? 4 : (lanes * 2 <= T ? 2 : 1);
        for (int cap : {forward_cap, tuning.max_split_adjoint}) {
            if (tuning.scaled && cap == forward_cap && cap != tuning.max_split_adjoint) continue;
            const int g = std::min(G, cap);
            if (std::find(splits.begin(), splits.end(), g) == splits.end()) splits.push_back(g);
        }
    }
    for (int G : splits)
        if (G > 1) o << "#define CPDE_SPLIT" << G << " 1\n";
    o << compose_source(t, splits, tuning.scaled != 0);
    o << kFusedSource;
}

// Body of a one-pass epoch kernel: the forward of the workgroup's points, the
// output values and the output adjoint of its columns kept in LDS (O), the
// cost stage `cost` between them (it fills O's second half), then the
// backward.  The row-major weight copies are written before the launch.
static std::string epoch_body(const std::vector<int>& neurons, const std::string& prefetch, const std::string& cost,
                              bool stamps, const std::string& after_input = "") {
    const int L = int(neurons.size()), NO = neurons[L - 1];
    std::ostringstream ep;
    // S: the cost stage's scratch (matching terms, or a double and an int per
    // point of an expression), T itself unless T is the operand tile X, which
    // holds the last hidden layer's values until the output backward
    const std::string scratch = "(kNNC * " + std::to_string(NO) + " > 4 * kNPB ? kNNC * " + std::to_string(NO) +
                                " : 4 * kNPB)";
    // The grids have one block per kNPB points of the chunk's width, so at one
    // point per block every block has its point: npts is the constant 1 there,
    // which leaves the phases' loops and the products' column checks to the
    // compiler.
    ep << tile_declarations()
       << "    __shared__ __attribute__((aligned(16))) float O[2 * kNNC * " << NO << "];\n"
       << "#ifdef CPDE_ALIAS_TILES\n"
       << "    __shared__ __attribute__((aligned(16))) float S[" << scratch << "];\n"
       << "#else\n"
       << "    float* const S = T;\n"
       << "#endif\n"
       << "    const int p0 = net_block(a) * kNPB, npts = kNPB == 1 ? 1 : min(kNPB, points - p0);\n"
       << "    tier_priority(a, 0);\n"
       << prefetch << "    const float xin = input_ahead<" << neurons[0] << ">(a, p0, npts);  // for the input gradient\n"
       << "    net_input<" << neurons[0] << ", " << neurons[1] << ">(a, X, p0, npts);\n"
       << "    zero_pad(X, " << neurons[1] << ", " << (neurons[1] + 7) / 8 * 8 << ");\n"
       << "    __syncthreads();\n"
       << after_input;
    // the last hidden layer's y (read from X by the output layer's partial) and
    // the first one's dE/dz (read from X by the input transition's) stay in the
    // workgroup: no later launch reads them
    int marker = 0;
    for (int t = 1; t + 2 < L; ++t)
        ep << "    tier_priority(a, " << ++marker << ");\n"
           << "    net_hidden<" << neurons[t] << ", " << neurons[t + 1] << (t + 3 == L ? ", false" : "") << ">(a, " << t
           << ", X, T, p0, npts);\n";
    const std::string last = std::to_string(neurons[L - 2]);
    ep << "    tier_priority(a, " << ++marker << ");\n";
    ep << "    UAhead<" << last << ", output_adjoint_split<" << last
       << ">()> ua;  // the last hidden layer's u rows, in flight during the output layer and the cost\n"
       << "    u_ahead<" << last << ", output_adjoint_split<" << last << ">()>(a, " << L - 2 << ", p0, npts, ua);\n"
       << "    WAhead<" << last << ", " << NO << "> wa;  // and the output weights of the lane's adjoint items\n"
       << "    w_ahead<" << last << ", " << NO << ">(a, " << L - 2 << ", npts, wa);\n"
       << "    net_output<" << neurons[L - 2] << ", " << NO << ">(a, " << L - 2 << ", X, p0, npts, O);\n"
       << "    __syncthreads();  // the output values of the block's columns are in O\n"
       << "    tier_priority(a, " << ++marker << ");\n"
       << cost << "    net_output_backward<" << neurons[L - 2] << ", " << NO << ", true>(a, " << L - 2
       << ", X, p0, npts, ua, O + kNNC * " << NO << ", &wa);\n";
    for (int t = L - 3; t >= 1; --t)
        ep << "    tier_priority(a, " << ++marker << ");\n"
           << "    net_hidden_backward<" << neurons[t] << ", " << neurons[t + 1] << (t == 1 ? ", false" : "") << ">(a, "
           << t << ", X, T, p0, npts);\n";
    ep << "    net_input_gradient<" << neurons[0] << ", " << neurons[1] << ", true>(a, X, p0, npts, xin);\n";
    // Diagnostics (FusedTuning::stamps): a clock stamp after every phase --
    // each call above and each barrier between them -- written over the
    // block's output stack when the epoch ends.
    if (!stamps) return ep.str();
    std::istringstream lines(ep.str());
    std::ostringstream st;
    std::string line;
    int k = 0;
    bool begun = false;
    while (std::getline(lines, line)) {
        st << line << "\n";
        if (!begun && line.find("const int p0") != std::string::npos) {
            st << "    STAMP_BEGIN\n";
            begun = true;
        } else if (begun && (line.rfind("    net_", 0) == 0 || line.rfind("    __syncthreads();", 0) == 0)) {
            st << "    STAMP(" << k++ << ")\n";
        }
    }
    st << "    STAMP_END(" << k << ", a.Z[" << L - 1 << "] + size_t(p0) * R * " << NO << ", R * " << NO
       << " * npts)\n";
    return st.str();
}

// Full source of the fused module for a schema and architecture.
std::string fused_source(const Tables& t, const std::vector<int>& neurons, const FusedTuning& tuning) {
    std::ostringstream o;
    const int L = int(neurons.size());
    emit_prologue(o, t, neurons, tuning);
    // network-fused forward and backward, one call per layer with its widths;
    // the one-pass epoch runs both with the matching cost between them
    std::ostringstream fwd, bwd;
    fwd << "    const int p0 = net_block(a) * kNPB, npts = kNPB == 1 ? 1 : min(kNPB, points - p0);\n";
    for (int t = 1; t + 2 < L; ++t)
        fwd << "    net_transpose<" << neurons[t] << ", " << neurons[t + 1] << ">(a, " << t << ");\n";
    fwd << "    net_input<" << neurons[0] << ", " << neurons[1] << ">(a, X, p0, npts);\n"
        << "    zero_pad(X, " << neurons[1] << ", " << (neurons[1] + 7) / 8 * 8 << ");\n"
        << "    __syncthreads();\n";
    for (int t = 1; t + 2 < L; ++t)
        fwd << "    net_hidden<" << neurons[t] << ", " << neurons[t + 1] << ">(a, " << t << ", X, T, p0, npts);\n";
    fwd << "    net_output<" << neurons[L - 2] << ", " << neurons[L - 1] << ">(a, " << L - 2 << ", X, p0, npts);\n";
    {
        const std::string last = std::to_string(neurons[L - 2]);
        bwd << "    UAhead<" << last << ", output_adjoint_split<" << last << ">()> ua;\n    u_ahead<" << last
            << ", output_adjoint_split<" << last << ">()>(a, " << L - 2
            << ", p0, npts, ua);\n"
            << "    net_output_backward<" << neurons[L - 2] << ", " << neurons[L - 1] << ">(a, " << L - 2
            << ", X, p0, npts, ua);\n";
    }
    for (int t = L - 3; t >= 1; --t)
        bwd << "    net_hidden_backward<" << neurons[t] << ", " << neurons[t + 1] << ">(a, " << t << ", X, T, p0, npts);\n";
    bwd << "    net_input_gradient<" << neurons[0] << ", " << neurons[1] << ">(a, X, p0, npts);\n";
    const std::string tiles = tile_declarations();
    const std::string nt = std::to_string(tuning.net_threads);
    o << "\nextern \"C\" __global__ __launch_bounds__(" << nt << ", " << tuning.forward_blocks
      << ") void network_forward_k(NetArgs a, int points) {\n"
      << tiles << fwd.str() << "}\n";
    o << "extern \"C\" __global__ __launch_bounds__(" << nt << ", " << tuning.backward_blocks
      << ") void network_backward_k(NetArgs a, int points) {\n"
      << tiles << "    const int p0 = net_block(a) * kNPB, npts = kNPB == 1 ? 1 : min(kNPB, points - p0);\n" << bwd.str() << "}\n";
    {
        const int NO = neurons[L - 1];
        const std::string prefetch =
            "    const MatchAhead pa = match_ahead<" + std::to_string(NO) + ">(m, p0, npts);\n";
        const std::string after_input =
            "    const MatchTerm pre = match_fetch<" + std::to_string(NO) + ">(m, p0, npts, pa);\n";
        const std::string cost = "    net_match<" + std::to_string(NO) + ">(a, m, " + std::to_string(L - 1) +
                                 ", S, p0, npts, O, O + kNNC * " + std::to_string(NO) + ", pre);\n";
        o << "extern \"C\" __global__ __launch_bounds__(" << nt << ", " << tuning.backward_blocks
          << ") void network_epoch_k(NetArgs a, MatchArgs m, int points) {\n"
          << epoch_body(neurons, prefetch, cost, tuning.stamps != 0, after_input) << "}\n";
    }
    o << "\nextern \"C\" __global__ __launch_bounds__(256) void input_layer_k(const float* W, const float* X, float* Z,"
         " float* Y, int points) { input_layer<"
      << neurons[0] << ", " << neurons[1] << ">(W, X, Z, Y, points); }\n";
    for (int t = 1; t + 2 < L; ++t) {
        o << "extern \"C\" __global__ __launch_bounds__(256) void hidden_forward_" << t
          << "(const float* W, const float* Yin, float* Z, float* Yout, int points) { hidden_forward<" << neurons[t]
          << ", " << neurons[t + 1] << ">(W, Yin, Z, Yout, points); }\n";
        o << "extern \"C\" __global__ __launch_bounds__(256) void hidden_backward_" << t
          << "(const float* W, const float* Gnext, const float* Zl, float* Gl, int points) { hidden_backward<"
          << neurons[t] << ", " << neurons[t + 1] << ">(W, Gnext, Zl, Gl, points); }\n";
    }
    o << "extern \"C\" __global__ __launch_bounds__(256) void output_backward_k(const float* W, const float* G,"
         " const float* Zl, float* Gl, int points) { output_backward<"
      << neurons[L - 2] << ", " << neurons[L - 1] << ">(W, G, Zl, Gl, points); }\n";
    return o.str();
}

// The expression cost's stage of a one-pass epoch, and the fetch of its
// inputs when the epoch starts.
static std::string expression_cost(int L, int NO) {
    return "    net_expression<" + std::to_string(NO) + ">(a, e, " + std::to_string(L - 1) +
           ", S, p0, npts, O, O + kNNC * " + std::to_string(NO) + ", ahead);\n";
}
static std::string expression_ahead_line() {
    return "    const ExpressionAhead ahead = expression_ahead(e, p0, npts);\n";
}

// The one-pass epoch of an expression cost: the expression program (which
// defines cpde_expression_inputs and cpde_expression_point) compiled together
// with the network kernels of a schema and architecture.
std::string expression_epoch_source(const Tables& t, const std::vector<int>& neurons, const FusedTuning& tuning,
                                    const std::string& program) {
    std::ostringstream o;
    const int L = int(neurons.size()), NO = neurons[L - 1];
    o << "// generated: one-pass epoch of an expression cost\n" << program << "\n#define CPDE_EXPRESSION_EPOCH 1\n";
    emit_prologue(o, t, neurons, tuning);
    o << "extern \"C\" __global__ __launch_bounds__(" << tuning.net_threads << ", " << tuning.backward_blocks
      << ") void network_epoch_expression_k(NetArgs a, ExpressionArgs e, int points) {\n"
      << epoch_body(neurons, expression_ahead_line(), expression_cost(L, NO), tuning.stamps != 0) << "}\n";
    return o.str();
}

// Two one-pass expression epochs over one network in one launch: each leaf's
// program, tuning macros, compositions and device code in a namespace of its
// own (its macros undefined after it, so the next leaf defines its own; the
// program's kernel named `expression` renamed per leaf), and a
// kernel whose workgroups below the second leaf's block offset run the first
// leaf's epoch and the rest the second's.  Both leaves need the same threads
// per workgroup.
std::string expression_pair_source(const Tables& t0, const FusedTuning& u0, const std::string& program0,
                                   const Tables& t1, const FusedTuning& u1, const std::string& program1,
                                   const std::vector<int>& neurons) {
    if (u0.net_threads != u1.net_threads) throw std::runtime_error("paired epochs need equal workgroup sizes");
    std::ostringstream o;
    const int L = int(neurons.size()), NO = neurons[L - 1];
    o << "// generated: two one-pass epochs of expression costs in one launch\n";
    const std::string cost = expression_cost(L, NO);
    for (int leaf = 0; leaf < 2; ++leaf) {
        std::ostringstream part;
        // the program's stand-alone cost kernel has C linkage, which the
        // namespace does not scope: each leaf's gets a name of its own
        part << "#define expression cpde_leaf" << leaf << "_expression\n"
             << (leaf ? program1 : program0) << "\n#undef expression\n#define CPDE_EXPRESSION_EPOCH 1\n";
        emit_prologue(part, leaf ? t1 : t0, neurons, leaf ? u1 : u0);
        part << "__device__ __forceinline__ void epoch(const NetArgs& a, const ExpressionArgs& e, int points) {\n"
             << epoch_body(neurons, expression_ahead_line(), cost, (leaf ? u1 : u0).stamps != 0) << "}\n";
        const std::string text = part.str();
        o << "namespace cpde_leaf" << leaf << " {\n" << text << "}  // namespace cpde_leaf" << leaf << "\n";
        std::istringstream lines(text);
        std::string line;
        while (std::getline(lines, line)) {
            const size_t at = line.find_first_not_of(" \t");
            if (at == std::string::npos || line.compare(at, 7, "#define") != 0) continue;
            std::istringstream words(line.substr(at + 7));
            std::string name;
            words >> name;
            o << "#undef " << name << "\n";
        }
    }
    o << "extern \"C\" __global__ __launch_bounds__(" << u0.net_threads << ", "
      << std::max(u0.backward_blocks, u1.backward_blocks)
      << ") void network_epoch_pair_k(cpde_leaf0::NetArgs a0, cpde_leaf0::ExpressionArgs e0, int points0,"
         " cpde_leaf1::NetArgs a1, cpde_leaf1::ExpressionArgs e1, int points1) {\n"
         "    if (int(blockIdx.x) < a1.block_offset) cpde_leaf0::epoch(a0, e0, points0);\n"
         "    else cpde_leaf1::epoch(a1, e1, points1);\n"
         "}\n";
    return o.str();
}

}  // namespace cpde
