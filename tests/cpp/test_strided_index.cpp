// test_strided_index.cpp — CPU check of the index arithmetic the strided
// kernels run (csrc/strided_index.hpp): multiply-high division against
// hardware division, and the axis merge against a plain multi-axis walk,
// by replaying the kernels' per-unit offset computation on the host.
// Exit status 0 and a last line "OK" when every check passes.
#include <algorithm>
#include <cstdio>
#include <random>
#include <vector>

#include "strided_index.hpp"

using namespace msst;

static int g_fail = 0;
#define EXPECT(c, ...)                    \
    do {                                  \
        if (!(c)) {                       \
            ++g_fail;                     \
            std::printf("FAIL: " __VA_ARGS__); \
            std::printf("\n");            \
        }                                 \
    } while (0)

static void check_div(uint64_t d, uint64_t n) {
    const FastDiv f = make_fastdiv(d);
    uint64_t q;
    const uint64_t r = f.divmod(n, &q);
    EXPECT(q == n / d && r == n % d, "%llu / %llu: got q=%llu r=%llu", (unsigned long long)n,
           (unsigned long long)d, (unsigned long long)q, (unsigned long long)r);
}

// Offsets (src, dst) of every unit in kernel order, from the merged axes.
static void kernel_offsets(const MergedAxes& m, std::vector<int64_t>& so, std::vector<int64_t>& dof) {
    IndexSpace sp;
    uint64_t total = 0;
    make_index_space(m, sp, total);
    so.resize(total);
    dof.resize(total);
    for (uint64_t i = 0; i < total; ++i) {
        int64_t a = 0, b = 0;
        uint64_t rem = i;
        for (int d = kMaxDims - 1; d >= 0; --d) {
            if (d < sp.ndim) {
                uint64_t q;
                const uint64_t c = sp.div[d].divmod(rem, &q);
                rem = q;
                a += (int64_t)c * m.stride[0][d];
                b += (int64_t)c * m.stride[1][d];
            }
        }
        so[i] = a;
        dof[i] = b;
    }
}

// Offsets of every index in row-major order of the original axes.
static void naive_offsets(const std::vector<int64_t>& shape, const std::vector<int64_t>& ss,
                          const std::vector<int64_t>& ds, std::vector<int64_t>& so,
                          std::vector<int64_t>& dof) {
    const int n = (int)shape.size();
    int64_t total = 1;
    for (int64_t s : shape) total *= s;
    so.clear();
    dof.clear();
    std::vector<int64_t> c(n, 0);
    for (int64_t i = 0; i < total; ++i) {
        int64_t a = 0, b = 0;
        for (int d = 0; d < n; ++d) {
            a += c[d] * ss[d];
            b += c[d] * ds[d];
        }
        so.push_back(a);
        dof.push_back(b);
        for (int d = n - 1; d >= 0; --d) {
            if (++c[d] < shape[d]) break;
            c[d] = 0;
        }
    }
}

int main() {
    // Division: small divisors exhaustively over small n, powers of two and
    // their neighbours, extremes, random pairs.
    for (uint64_t d = 1; d <= 600; ++d)
        for (uint64_t n = 0; n < 3000; n += 1 + (n % 7)) check_div(d, n);
    for (int k = 0; k < 64; ++k) {
        const uint64_t p = (uint64_t)1 << k;
        for (uint64_t d : {p, p - 1, p + 1})
            if (d >= 1)
                for (uint64_t n : {(uint64_t)0, (uint64_t)1, d - 1, d, d + 1, 2 * d, ~(uint64_t)0,
                                   ~(uint64_t)0 - 1, ((uint64_t)1 << 62) + 12345})
                    check_div(d, n);
    }
    std::mt19937_64 g(7);
    for (int i = 0; i < 200000; ++i) {
        const uint64_t d = 1 + (g() >> (g() % 64));
        check_div(d, g() >> (g() % 64));
    }

    // Views: random permutations / slices / broadcasts of random shapes;
    // the merged kernel walk must visit the same (src, dst) pairs in the same
    // order as the plain walk.
    int cases = 0;
    for (int it = 0; it < 3000; ++it) {
        const int n = 1 + (int)(g() % 6);
        std::vector<int64_t> shape(n), base(n);
        for (int d = 0; d < n; ++d) base[d] = 1 + (int64_t)(g() % 5);
        // source: row-major strides of `base`, then a permutation, a slice
        // or a broadcast (stride 0) applied per axis
        std::vector<int64_t> rs(n);
        int64_t acc = 1;
        for (int d = n - 1; d >= 0; --d) {
            rs[d] = acc;
            acc *= base[d];
        }
        std::vector<int> perm(n);
        for (int d = 0; d < n; ++d) perm[d] = d;
        if (g() % 2) std::shuffle(perm.begin(), perm.end(), g);
        std::vector<int64_t> ss(n);
        for (int d = 0; d < n; ++d) {
            shape[d] = base[perm[d]];
            ss[d] = rs[perm[d]];
            const int kind = (int)(g() % 5);
            if (kind == 0 && shape[d] > 1) shape[d] -= 1;       // slice
            if (kind == 1) { ss[d] = 0; shape[d] = 1 + g() % 4; }  // broadcast
        }
        // destination: row-major over `shape`, or a slab of a wider tensor
        std::vector<int64_t> ds(n);
        acc = 1;
        const int wide = (int)(g() % n);
        for (int d = n - 1; d >= 0; --d) {
            ds[d] = acc;
            acc *= shape[d] + (d == wide && (g() % 2) ? 3 : 0);
        }
        const MergedAxes m = merge_axes(shape.data(), n, {ss.data(), ds.data()});
        if (m.empty) continue;
        std::vector<int64_t> ka, kb, na, nb;
        kernel_offsets(m, ka, kb);
        naive_offsets(shape, ss, ds, na, nb);
        EXPECT(ka == na && kb == nb, "case %d: merged walk differs (ndim %d -> %d)", it, n, m.ndim);
        ++cases;
    }
    // Zero extents are empty; all-ones shapes keep one unit.
    const int64_t z[3] = {2, 0, 3}, s3[3] = {3, 3, 1};
    EXPECT(merge_axes(z, 3, {s3, s3}).empty, "zero extent not empty");
    const int64_t o[2] = {1, 1}, s2[2] = {5, 7};
    const MergedAxes mo = merge_axes(o, 2, {s2, s2});
    EXPECT(!mo.empty && mo.ndim == 1 && mo.shape[0] == 1, "all-ones shape");
    std::printf("%d view cases\n", cases);
    if (g_fail) {
        std::printf("%d failures\n", g_fail);
        return 1;
    }
    std::printf("OK\n");
    return 0;
}
