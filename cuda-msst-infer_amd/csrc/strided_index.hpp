// strided_index.hpp — index-space helpers of the strided kernels
// (strided.hip), usable on the host (where they are unit-tested on the CPU)
// and on the device.
//
// FastDiv: n / d for 64-bit n by an invariant d >= 1 with one multiply-high
// (Granlund & Montgomery, PLDI 1994, "round-up" method): with
// l = ceil(log2 d) and m = floor(2^64 (2^l - d) / d) + 1,
//   t = mulhi(m, n),  q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0).
// MergedAxes: a shape and up to three stride sets with size-1 axes dropped
// and adjacent axes merged wherever every stride set is contiguous across
// them (outer stride == inner stride * inner extent).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

namespace msst {

constexpr int kMaxDims = 8;

struct FastDiv {
    uint64_t d, m;
    uint32_t sh1, sh2;

    __host__ __device__ static uint64_t mulhi(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
        return __umul64hi(a, b);
#else
        return (uint64_t)(((unsigned __int128)a * b) >> 64);
#endif
    }
    __host__ __device__ uint64_t quot(uint64_t n) const {
        const uint64_t t = mulhi(m, n);
        return (t + ((n - t) >> sh1)) >> sh2;
    }
    // n = q * d + r; returns r, q in *q.
    __host__ __device__ uint64_t divmod(uint64_t n, uint64_t* q) const {
        *q = quot(n);
        return n - *q * d;
    }
};

inline FastDiv make_fastdiv(uint64_t d) {
    uint32_t l = 0;
    while (l < 64 && ((uint64_t)1 << l) < d) ++l;  // l = ceil(log2 d), d >= 1
    FastDiv f;
    f.d = d;
    const unsigned __int128 two_l = (unsigned __int128)1 << l;
    f.m = (uint64_t)(((unsigned __int128)1 << 64) * (two_l - d) / d) + 1;
    f.sh1 = l < 1 ? l : 1;
    f.sh2 = l > 1 ? l - 1 : 0;
    return f;
}

struct IndexSpace {
    int ndim;
    FastDiv div[kMaxDims];  // extents, innermost axis last
};

struct MergedAxes {
    bool empty = false;
    int ndim = 0;
    int64_t shape[kMaxDims] = {};
    int64_t stride[3][kMaxDims] = {};
    int nsets = 0;
};

// Drops size-1 axes and merges contiguous neighbours.  empty: some extent
// is 0 (nothing to do).  At least one axis remains.
inline MergedAxes merge_axes(const int64_t* shape, int ndim,
                             std::initializer_list<const int64_t*> strides) {
    MergedAxes m;
    m.nsets = (int)strides.size();
    for (int d = 0; d < ndim; ++d)
        if (shape[d] == 0) m.empty = true;
    if (m.empty) return m;
    for (int d = 0; d < ndim; ++d) {
        if (shape[d] == 1) continue;
        int k = 0;
        bool merge = m.ndim > 0;
        for (const int64_t* s : strides) {
            if (merge && m.stride[k][m.ndim - 1] != s[d] * shape[d]) merge = false;
            ++k;
        }
        if (merge) {
            // Outer axis (already in m) absorbs axis d: extent multiplies,
            // strides become the inner ones.
            m.shape[m.ndim - 1] *= shape[d];
            k = 0;
            for (const int64_t* s : strides) m.stride[k++][m.ndim - 1] = s[d];
        } else {
            m.shape[m.ndim] = shape[d];
            k = 0;
            for (const int64_t* s : strides) m.stride[k++][m.ndim] = s[d];
            ++m.ndim;
        }
    }
    if (m.ndim == 0) {
        m.ndim = 1;
        m.shape[0] = 1;
    }
    return m;
}

// The merged axes as a device index space; false if the element count
// reaches 2^62.
inline bool make_index_space(const MergedAxes& m, IndexSpace& sp, uint64_t& total) {
    sp.ndim = m.ndim;
    total = 1;
    for (int d = 0; d < m.ndim; ++d) {
        if ((uint64_t)m.shape[d] > ((uint64_t)1 << 62) / total) return false;
        total *= (uint64_t)m.shape[d];
        sp.div[d] = make_fastdiv((uint64_t)m.shape[d]);
    }
    for (int d = m.ndim; d < kMaxDims; ++d) sp.div[d] = make_fastdiv(1);
    return true;
}

}  // namespace msst
