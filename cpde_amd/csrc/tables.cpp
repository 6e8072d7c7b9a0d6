// Host construction of the composition term tables for one derivative schema.
//
// The reference enumerates, per row of order k, the 2^k subsets of the row's
// direction list and hard-codes every set partition of them in d1..d6 /
// d1p..d6p (cuda/cpde_engine.cuh:391-457, cuda/derivative_kernels_v4.cu:12-745).
// Here the set partitions are enumerated once on the host and grouped by the
// multiset of block rows they produce: partitions that multiply the same stack
// rows collapse into one term with an integer coefficient (1837 set-partition
// terms become 275 multiset terms for two variables through order 6).  The
// adjoint pairs follow derivative_tables (cuda/cpde_engine.cuh:476-498).
#include <algorithm>
#include <array>
#include <cstring>
#include <map>

#include "common.hpp"

namespace cpde {

namespace {

int find_row(const std::vector<int>& table, int rows, int variables, const int* counts) {
    for (int r = 0; r < rows; ++r) {
        bool ok = true;
        for (int v = 0; v < variables && ok; ++v) ok = table[r * (variables + 1) + 1 + v] == counts[v];
        if (ok) return r;
    }
    return -1;
}

int binomial(int a, int b) {
    if (b < 0 || b > a) return 0;
    int r = 1;
    for (int i = 1; i <= b; ++i) r = r * (a - b + i) / i;
    return r;
}

struct Enumerator {
    const std::vector<int>& table;
    int rows, variables, k;
    int dirs[kMaxOrder];
    int rgs[kMaxOrder];
    // (m, sorted block rows) -> number of set partitions
    std::map<std::pair<int, std::array<int, kMaxOrder>>, int> terms;

    void run(int pos, int maxlab) {
        if (pos == k) {
            int m = maxlab + 1;
            std::array<int, kMaxOrder> blocks{};
            blocks.fill(-1);
            for (int b = 0; b < m; ++b) {
                int counts[32] = {0};
                for (int q = 0; q < k; ++q)
                    if (rgs[q] == b) counts[dirs[q]]++;
                int row = find_row(table, rows, variables, counts);
                require(row >= 0, "derivative closure is missing a sub-derivative");
                blocks[b] = row;
            }
            std::sort(blocks.begin(), blocks.begin() + m);
            terms[{m, blocks}] += 1;
            return;
        }
        for (int lab = 0; lab <= maxlab + 1; ++lab) {
            rgs[pos] = lab;
            run(pos + 1, std::max(lab, maxlab));
        }
    }
};

int float_bits(float f) {
    int i;
    std::memcpy(&i, &f, sizeof i);
    return i;
}

}  // namespace

Tables build_tables(int rows, int variables, const int* table) {
    require(rows > 0 && rows <= kMaxRows, "derivative schema must have 1..255 rows");
    require(variables > 0 && variables <= 26, "invalid variable count");
    Tables t;
    t.rows = rows;
    t.variables = variables;
    t.table.assign(table, table + size_t(rows) * (variables + 1));
    int previous = -1;
    for (int r = 0; r < rows; ++r) {
        int order = t.table[r * (variables + 1)], sum = 0;
        for (int v = 0; v < variables; ++v) {
            int c = t.table[r * (variables + 1) + 1 + v];
            require(c >= 0, "derivative counts must be nonnegative");
            sum += c;
        }
        require(sum == order, "derivative order must equal the sum of counts");
        require(order >= previous && order <= kMaxOrder, "derivative closure must be sorted, orders 0..6");
        previous = order;
        t.max_order = std::max(t.max_order, order);
    }
    require(t.table[0] == 0, "value derivative must come first");

    t.fwd_offset.assign(rows, -1);
    t.pair_offset.assign(rows, -1);
    for (int r = 1; r < rows; ++r) {
        Enumerator e{t.table, rows, variables, t.table[r * (variables + 1)], {}, {}, {}};
        int q = 0;
        for (int v = 0; v < variables; ++v)
            for (int c = 0; c < t.table[r * (variables + 1) + 1 + v]; ++c) e.dirs[q++] = v;
        e.rgs[0] = 0;
        e.run(1, 0);
        t.fwd_offset[r] = int(t.words.size());
        t.words.push_back(e.k);
        for (int m = 1; m <= e.k; ++m) {
            int count_pos = int(t.words.size());
            t.words.push_back(0);
            int count = 0;
            for (const auto& kv : e.terms) {
                if (kv.first.first != m) continue;
                int w0 = 0, w1 = 0;
                for (int b = 0; b < m; ++b) {
                    int row = kv.first.second[b];
                    if (b < 4) w0 |= row << (8 * b);
                    else w1 |= row << (8 * (b - 4));
                }
                t.words.push_back(float_bits(float(kv.second)));
                t.words.push_back(w0);
                t.words.push_back(w1);
                ++count;
            }
            t.words[count_pos] = count;
            t.forward_terms += count;
        }
    }
    for (int i = 0; i < rows; ++i) {
        t.pair_offset[i] = int(t.words.size());
        int count_pos = int(t.words.size());
        t.words.push_back(0);
        int count = 0;
        for (int j = i + 1; j < rows; ++j) {
            int diff[32];
            int coefficient = 1;
            bool ok = true;
            for (int v = 0; v < variables; ++v) {
                int a = t.table[j * (variables + 1) + 1 + v], b = t.table[i * (variables + 1) + 1 + v];
                diff[v] = a - b;
                if (a < b) ok = false;
                else coefficient *= binomial(a, b);
            }
            if (!ok) continue;
            int dn = find_row(t.table, rows, variables, diff);
            if (dn < 0) continue;
            t.words.push_back(j);
            t.words.push_back(dn);
            t.words.push_back(float_bits(float(coefficient)));
            ++count;
        }
        t.words[count_pos] = count;
        t.pair_terms += count;
    }
    return t;
}

}  // namespace cpde
