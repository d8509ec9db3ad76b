/* Internal interface between the HIP kernels (q8_kernels.hip) and the
 * runtime that exposes them through the C ABI (pk_hip.cpp). */
#ifndef PK_Q8_INTERNAL_H
#define PK_Q8_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pkq8 {

/* A matrix in HBM, repacked from PK_Q8 (16-row panels, groups of 4 inputs)
 * into units of 16 rows by 64 inputs: a unit is 1 KB, the 16 rows' 64 bytes
 * in the order the 16x16x64 int8 MFMA takes an operand (byte 16 * (kq * 16 +
 * r) + kb holds row r, input 16 * kq + kb of the unit), and a panel's ku =
 * ceil(cols / 64) units follow one another, inputs past cols zero. A panel
 * is therefore 1 KB * ku contiguous bytes, and any whole panel of the matrix
 * starts a valid matrix of fewer rows. */
constexpr uint32_t kUnitBytes = 1024;

inline uint32_t units_per_panel(uint32_t cols) { return (cols + 63) / 64; }

/* One segment of activations and outputs. */
struct Seg {
    float *out;
    const int8_t *q;
    const float *d;
    uint64_t os;
    uint32_t T;
    uint32_t tile0;             /* the grouped launch's first M tile of this segment */
};

constexpr int kMaxSegs = 64;

struct SegTable {
    Seg s[kMaxSegs];
    uint32_t nseg;
};

/* What every product launch shares. */
struct GemmArgs {
    const int8_t *w;            /* repacked weights, at the first panel of the call */
    const float *ws, *bias;     /* at the first row of the call */
    uint32_t rows;              /* N, a multiple of 16 */
    uint32_t n;                 /* K, a multiple of 32 */
    uint32_t ku;                /* units a panel */
    uint32_t qb, nb;            /* block inputs, blocks a column */
    int add;
    int rmode;                  /* 0 nearest, 1 upward, 2 downward, 3 toward zero */
};

int launch_repack(int8_t *dst, const int8_t *src, uint32_t rows, uint32_t cols, hipStream_t s);

int launch_quantize(int8_t *q, float *d, const float *x, size_t xs, uint32_t n, uint32_t qb,
                    uint32_t T, hipStream_t s, const char **name);

/* One product; table->nseg == 1 for a plain call. */
int launch_gemm(const GemmArgs &g, const SegTable &table, hipStream_t s, const char **name);

}  // namespace pkq8

#endif
