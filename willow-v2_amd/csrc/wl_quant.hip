// Q4_K / Q6_K dequantization and GEMV kernels, and their C-ABI entry points (include/willow_hip.h).
// Replaces the Metal kernels dequant_<T>, gemv_<T>, gemv_batch_<T>, gemv_combine_<T> (gguf/metal.py:189-291).
#include <hip/hip_runtime.h>

#include "wl_common.h"
#include "wl_host.h"

namespace wl {

// ---------------------------------------------------------------------------------------------------------------
// Dequantization: one lane per (row, block, lane-chunk); each lane writes its two runs of 16 values.
template <int TYPE, bool BF16>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ w, int64_t rows, int nb,
                                                 int64_t row_stride, void* __restrict__ out) {
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t unit = tid >> 3;
    if (unit >= rows * nb) return;
    const int c = static_cast<int>(tid & 7);
    const int64_t row = unit / nb;
    const int kb = static_cast<int>(unit - row * nb);
    Lane32 l;
    decode<TYPE>(w + row * row_stride + static_cast<int64_t>(kb) * BlockInfo<TYPE>::bytes, c, l);
    const int64_t base = row * static_cast<int64_t>(nb) * kQK + static_cast<int64_t>(kb) * kQK;
    const int64_t lo = base + BlockInfo<TYPE>::lo_start(c), hi = lo + BlockInfo<TYPE>::hi_offset;
    if constexpr (BF16) {
        uint32_t plo[8], phi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int wi = i >> 1, n = 2 * (i & 1);
            plo[i] = f32_to_bf16_bits(dequant_value<TYPE>(l.lo[wi], n, l.a_lo, l.b_lo)) |
                     (f32_to_bf16_bits(dequant_value<TYPE>(l.lo[wi], n + 1, l.a_lo, l.b_lo)) << 16);
            phi[i] = f32_to_bf16_bits(dequant_value<TYPE>(l.hi[wi], n, l.a_hi, l.b_hi)) |
                     (f32_to_bf16_bits(dequant_value<TYPE>(l.hi[wi], n + 1, l.a_hi, l.b_hi)) << 16);
        }
        uint4* olo = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + lo);
        uint4* ohi = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + hi);
        olo[0] = make_uint4(plo[0], plo[1], plo[2], plo[3]);
        olo[1] = make_uint4(plo[4], plo[5], plo[6], plo[7]);
        ohi[0] = make_uint4(phi[0], phi[1], phi[2], phi[3]);
        ohi[1] = make_uint4(phi[4], phi[5], phi[6], phi[7]);
    } else {
        float4* olo = reinterpret_cast<float4*>(static_cast<float*>(out) + lo);
        float4* ohi = reinterpret_cast<float4*>(static_cast<float*>(out) + hi);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            olo[i] = make_float4(dequant_value<TYPE>(l.lo[i], 0, l.a_lo, l.b_lo),
                                 dequant_value<TYPE>(l.lo[i], 1, l.a_lo, l.b_lo),
                                 dequant_value<TYPE>(l.lo[i], 2, l.a_lo, l.b_lo),
                                 dequant_value<TYPE>(l.lo[i], 3, l.a_lo, l.b_lo));
            ohi[i] = make_float4(dequant_value<TYPE>(l.hi[i], 0, l.a_hi, l.b_hi),
                                 dequant_value<TYPE>(l.hi[i], 1, l.a_hi, l.b_hi),
                                 dequant_value<TYPE>(l.hi[i], 2, l.a_hi, l.b_hi),
                                 dequant_value<TYPE>(l.hi[i], 3, l.a_hi, l.b_hi));
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// GEMV geometry: a wavefront's 8 lane groups take 8 blocks. With nb = k/256 blocks per row:
//   nb in {1, 2, 4}: the wave covers R = 8/nb whole rows at once (group g: row g/nb, block g%nb), and each row's
//                    partial sums are reduced over its 8*nb lanes;
//   otherwise:       one row per wave, group g takes blocks g, g+8, ...; reduction over all 64 lanes.
template <int WIDTH>
__device__ __forceinline__ float wsum(float v) {
    return group_sum<WIDTH>(v);
}

// y[t, r] = W[r, :] . x[t, :] for t < T <= TT.
template <int TYPE, int TT, int WIDTH>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ w, int rows, int nb, int64_t row_stride,
                                              const float* __restrict__ x, int T, int64_t ldx,
                                              float* __restrict__ y, int64_t ldy) {
    constexpr int R = WIDTH == 64 ? 1 : 64 / WIDTH;
    const int lane = threadIdx.x & 63;
    const int wave = static_cast<int>((static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6);
    const int nwaves = static_cast<int>((static_cast<int64_t>(gridDim.x) * blockDim.x) >> 6);
    const int g = lane >> 3, c = lane & 7;
    const int row_off = R > 1 ? g / nb : 0;
    const int kb0 = R > 1 ? g % nb : g;
    const int kb_step = R > 1 ? nb : 8;
    const bool slot_used = R > 1 ? (g < R * nb) : true;
    const int lo_start = BlockInfo<TYPE>::lo_start(c), hi_off = BlockInfo<TYPE>::hi_offset;
    for (int r0 = wave * R; r0 < rows; r0 += nwaves * R) {
        const int row = r0 + row_off;
        float acc[TT];
#pragma unroll
        for (int t = 0; t < TT; t++) acc[t] = 0.0f;
        if (slot_used && row < rows) {
            const uint8_t* rp = w + static_cast<int64_t>(row) * row_stride;
            for (int kb = kb0; kb < nb; kb += kb_step) {
                Lane32 l;
                decode<TYPE>(rp + static_cast<int64_t>(kb) * BlockInfo<TYPE>::bytes, c, l);
                const int lo = kb * kQK + lo_start;
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    if (t < T) {
                        float4 xl[4], xh[4];
                        load_run(x + t * ldx + lo, xl);
                        load_run(x + t * ldx + lo + hi_off, xh);
                        acc[t] += lane_dot(l, xl, xh);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const float s = wsum<WIDTH>(acc[t]);
            if (t < T && (lane & (WIDTH - 1)) == 0 && row < rows) y[t * ldy + row] = s;
        }
    }
}

// Batched experts, one token: grid.y = expert i; y[pos[i], r] = W_i[r, :] . x.
struct BatchTable {
    int64_t offset[WL_MAX_BATCH_EXPERTS];
    int64_t index[WL_MAX_BATCH_EXPERTS];
};

template <int TYPE, int WIDTH>
__global__ __launch_bounds__(256) void k_gemv_batch(const uint8_t* __restrict__ base, int rows, int nb,
                                                    int64_t row_stride, const float* __restrict__ x,
                                                    float* __restrict__ out, BatchTable tab) {
    constexpr int R = WIDTH == 64 ? 1 : 64 / WIDTH;
    const int e = blockIdx.y;
    const uint8_t* w = base + tab.offset[e];
    float* y = out + tab.index[e] * rows;
    const int lane = threadIdx.x & 63;
    const int wave = static_cast<int>((static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6);
    const int nwaves = static_cast<int>((static_cast<int64_t>(gridDim.x) * blockDim.x) >> 6);
    const int g = lane >> 3, c = lane & 7;
    const int row_off = R > 1 ? g / nb : 0;
    const int kb0 = R > 1 ? g % nb : g;
    const int kb_step = R > 1 ? nb : 8;
    const bool slot_used = R > 1 ? (g < R * nb) : true;
    const int lo_start = BlockInfo<TYPE>::lo_start(c), hi_off = BlockInfo<TYPE>::hi_offset;
    for (int r0 = wave * R; r0 < rows; r0 += nwaves * R) {
        const int row = r0 + row_off;
        float acc = 0.0f;
        if (slot_used && row < rows) {
            const uint8_t* rp = w + static_cast<int64_t>(row) * row_stride;
            for (int kb = kb0; kb < nb; kb += kb_step) {
                Lane32 l;
                decode<TYPE>(rp + static_cast<int64_t>(kb) * BlockInfo<TYPE>::bytes, c, l);
                float4 xl[4], xh[4];
                load_run(x + kb * kQK + lo_start, xl);
                load_run(x + kb * kQK + lo_start + hi_off, xh);
                acc += lane_dot(l, xl, xh);
            }
        }
        const float s = wsum<WIDTH>(acc);
        if ((lane & (WIDTH - 1)) == 0 && row < rows) y[row] = s;
    }
}

// y[r] = sum_i weights[perm[i]] * (W_i x_i)[r], in order of i (perm in tab.index).
template <int TYPE, int WIDTH>
__global__ __launch_bounds__(256) void k_gemv_combine(const uint8_t* __restrict__ base, int rows, int nb,
                                                      int64_t row_stride, const float* __restrict__ x, int k,
                                                      const float* __restrict__ weights, float* __restrict__ y,
                                                      int n, BatchTable tab) {
    constexpr int R = WIDTH == 64 ? 1 : 64 / WIDTH;
    const int lane = threadIdx.x & 63;
    const int wave = static_cast<int>((static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6);
    const int nwaves = static_cast<int>((static_cast<int64_t>(gridDim.x) * blockDim.x) >> 6);
    const int g = lane >> 3, c = lane & 7;
    const int row_off = R > 1 ? g / nb : 0;
    const int kb0 = R > 1 ? g % nb : g;
    const int kb_step = R > 1 ? nb : 8;
    const bool slot_used = R > 1 ? (g < R * nb) : true;
    const int lo_start = BlockInfo<TYPE>::lo_start(c), hi_off = BlockInfo<TYPE>::hi_offset;
    for (int r0 = wave * R; r0 < rows; r0 += nwaves * R) {
        const int row = r0 + row_off;
        float total = 0.0f;
        for (int i = 0; i < n; i++) {
            float acc = 0.0f;
            if (slot_used && row < rows) {
                const uint8_t* rp = base + tab.offset[i] + static_cast<int64_t>(row) * row_stride;
                const float* xi = x + static_cast<int64_t>(i) * k;
                for (int kb = kb0; kb < nb; kb += kb_step) {
                    Lane32 l;
                    decode<TYPE>(rp + static_cast<int64_t>(kb) * BlockInfo<TYPE>::bytes, c, l);
                    float4 xl[4], xh[4];
                    load_run(xi + kb * kQK + lo_start, xl);
                    load_run(xi + kb * kQK + lo_start + hi_off, xh);
                    acc += lane_dot(l, xl, xh);
                }
            }
            const float s = wsum<WIDTH>(acc);
            const float scaled = s * weights[tab.index[i]];
            total = i == 0 ? scaled : total + scaled;
        }
        if ((lane & (WIDTH - 1)) == 0 && row < rows) y[row] = total;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Host launchers

static int blocks_for_waves(int64_t waves) { return static_cast<int>((waves + 3) / 4); }

template <int TYPE, int TT>
static void launch_gemv_tt(const uint8_t* w, int rows, int nb, int64_t row_stride, const float* x, int T,
                           int64_t ldx, float* y, int64_t ldy, hipStream_t s) {
    const RowGeom geo = row_geom(nb);
    const int grid = blocks_for_waves((rows + geo.R - 1) / geo.R);
    switch (geo.width) {
        case 8: k_gemv<TYPE, TT, 8><<<grid, 256, 0, s>>>(w, rows, nb, row_stride, x, T, ldx, y, ldy); break;
        case 16: k_gemv<TYPE, TT, 16><<<grid, 256, 0, s>>>(w, rows, nb, row_stride, x, T, ldx, y, ldy); break;
        case 32: k_gemv<TYPE, TT, 32><<<grid, 256, 0, s>>>(w, rows, nb, row_stride, x, T, ldx, y, ldy); break;
        default: k_gemv<TYPE, TT, 64><<<grid, 256, 0, s>>>(w, rows, nb, row_stride, x, T, ldx, y, ldy); break;
    }
}

template <int TYPE>
static void launch_gemv(const uint8_t* w, int rows, int nb, int64_t row_stride, const float* x, int64_t tokens,
                        int64_t k, float* y, hipStream_t s) {
    for (int64_t t0 = 0; t0 < tokens; t0 += 8) {
        const int T = static_cast<int>(tokens - t0 < 8 ? tokens - t0 : 8);
        const float* xt = x + t0 * k;
        float* yt = y + t0 * rows;
        if (T == 1)
            launch_gemv_tt<TYPE, 1>(w, rows, nb, row_stride, xt, T, k, yt, rows, s);
        else if (T == 2)
            launch_gemv_tt<TYPE, 2>(w, rows, nb, row_stride, xt, T, k, yt, rows, s);
        else if (T <= 4)
            launch_gemv_tt<TYPE, 4>(w, rows, nb, row_stride, xt, T, k, yt, rows, s);
        else
            launch_gemv_tt<TYPE, 8>(w, rows, nb, row_stride, xt, T, k, yt, rows, s);
    }
}

template <int TYPE>
static void launch_gemv_batch(const uint8_t* base, int rows, int nb, int64_t row_stride, const float* x,
                              float* out, const BatchTable& tab, int n, hipStream_t s) {
    const RowGeom geo = row_geom(nb);
    const dim3 grid(blocks_for_waves((rows + geo.R - 1) / geo.R), n);
    switch (geo.width) {
        case 8: k_gemv_batch<TYPE, 8><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, out, tab); break;
        case 16: k_gemv_batch<TYPE, 16><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, out, tab); break;
        case 32: k_gemv_batch<TYPE, 32><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, out, tab); break;
        default: k_gemv_batch<TYPE, 64><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, out, tab); break;
    }
}

template <int TYPE>
static void launch_gemv_combine(const uint8_t* base, int rows, int nb, int64_t row_stride, const float* x,
                                int k, const float* weights, float* y, const BatchTable& tab, int n,
                                hipStream_t s) {
    const RowGeom geo = row_geom(nb);
    const int grid = blocks_for_waves((rows + geo.R - 1) / geo.R);
    switch (geo.width) {
        case 8:
            k_gemv_combine<TYPE, 8><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, k, weights, y, n, tab);
            break;
        case 16:
            k_gemv_combine<TYPE, 16><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, k, weights, y, n, tab);
            break;
        case 32:
            k_gemv_combine<TYPE, 32><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, k, weights, y, n, tab);
            break;
        default:
            k_gemv_combine<TYPE, 64><<<grid, 256, 0, s>>>(base, rows, nb, row_stride, x, k, weights, y, n, tab);
            break;
    }
}

}  // namespace wl

using namespace wl;

extern "C" {

int64_t wl_row_bytes(int type, int64_t k) {
    const int bb = block_bytes(type);
    if (bb < 0) return WL_EINVAL_TYPE;
    if (k <= 0 || k % kQK != 0) return WL_EINVAL_SHAPE;
    return k / kQK * bb;
}

int wl_dequant(int type, const void* w, int64_t rows, int64_t k, int64_t row_stride, int out_dtype, void* out,
               void* stream) {
    int rc = check_matrix(type, w, rows, k, row_stride);
    if (rc) return rc;
    if (!out) return WL_EINVAL_NULL;
    if (out_dtype != WL_DTYPE_F32 && out_dtype != WL_DTYPE_BF16) return WL_EINVAL_DTYPE;
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return WL_EINVAL_ALIGN;
    const int nb = static_cast<int>(k / kQK);
    const int64_t threads = rows * nb * 8;
    const int grid = static_cast<int>((threads + 255) / 256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (type == WL_TYPE_Q4_K) {
        if (out_dtype == WL_DTYPE_BF16)
            k_dequant<WL_TYPE_Q4_K, true><<<grid, 256, 0, s>>>(wb, rows, nb, row_stride, out);
        else
            k_dequant<WL_TYPE_Q4_K, false><<<grid, 256, 0, s>>>(wb, rows, nb, row_stride, out);
    } else {
        if (out_dtype == WL_DTYPE_BF16)
            k_dequant<WL_TYPE_Q6_K, true><<<grid, 256, 0, s>>>(wb, rows, nb, row_stride, out);
        else
            k_dequant<WL_TYPE_Q6_K, false><<<grid, 256, 0, s>>>(wb, rows, nb, row_stride, out);
    }
    return launch_status();
}

int wl_gemv(int type, const void* w, int64_t rows, int64_t k, int64_t row_stride, const float* x, int64_t tokens,
            float* y, void* stream) {
    int rc = check_matrix(type, w, rows, k, row_stride);
    if (rc) return rc;
    if (!x || !y) return WL_EINVAL_NULL;
    if (tokens <= 0) return WL_EINVAL_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return WL_EINVAL_ALIGN;
    const int nb = static_cast<int>(k / kQK);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (type == WL_TYPE_Q4_K)
        launch_gemv<WL_TYPE_Q4_K>(wb, static_cast<int>(rows), nb, row_stride, x, tokens, k, y, s);
    else
        launch_gemv<WL_TYPE_Q6_K>(wb, static_cast<int>(rows), nb, row_stride, x, tokens, k, y, s);
    return launch_status();
}

static int fill_table(int type, const void* base, int64_t rows, int64_t k, const int64_t* offsets,
                      const int64_t* index, int n, BatchTable& tab) {
    int rc = check_matrix(type, base, rows, k, wl_row_bytes(type, k));
    if (rc) return rc;
    if (!offsets || !index) return WL_EINVAL_NULL;
    if (n < 1 || n > WL_MAX_BATCH_EXPERTS) return WL_EINVAL_COUNT;
    const int64_t align = type == WL_TYPE_Q4_K ? 16 : 4;
    for (int i = 0; i < n; i++) {
        if (offsets[i] < 0 || offsets[i] % align != 0) return WL_EINVAL_ALIGN;
        if (index[i] < 0) return WL_EINVAL_SHAPE;
        tab.offset[i] = offsets[i];
        tab.index[i] = index[i];
    }
    return WL_OK;
}

int wl_gemv_batch(int type, const void* base, int64_t rows, int64_t k, const int64_t* offsets_host,
                  const int64_t* positions_host, int n, const float* x, float* out, void* stream) {
    BatchTable tab;
    int rc = fill_table(type, base, rows, k, offsets_host, positions_host, n, tab);
    if (rc) return rc;
    if (!x || !out) return WL_EINVAL_NULL;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return WL_EINVAL_ALIGN;
    const int nb = static_cast<int>(k / kQK);
    const int64_t rs = wl_row_bytes(type, k);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* bb = static_cast<const uint8_t*>(base);
    if (type == WL_TYPE_Q4_K)
        launch_gemv_batch<WL_TYPE_Q4_K>(bb, static_cast<int>(rows), nb, rs, x, out, tab, n, s);
    else
        launch_gemv_batch<WL_TYPE_Q6_K>(bb, static_cast<int>(rows), nb, rs, x, out, tab, n, s);
    return launch_status();
}

int wl_gemv_combine(int type, const void* base, int64_t rows, int64_t k, const int64_t* offsets_host,
                    const int64_t* perm_host, int n, const float* x, const float* weights, float* y,
                    void* stream) {
    BatchTable tab;
    int rc = fill_table(type, base, rows, k, offsets_host, perm_host, n, tab);
    if (rc) return rc;
    if (!x || !weights || !y) return WL_EINVAL_NULL;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return WL_EINVAL_ALIGN;
    const int nb = static_cast<int>(k / kQK);
    const int64_t rs = wl_row_bytes(type, k);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* bb = static_cast<const uint8_t*>(base);
    if (type == WL_TYPE_Q4_K)
        launch_gemv_combine<WL_TYPE_Q4_K>(bb, static_cast<int>(rows), nb, rs, x, static_cast<int>(k), weights, y,
                                          tab, n, s);
    else
        launch_gemv_combine<WL_TYPE_Q6_K>(bb, static_cast<int>(rows), nb, rs, x, static_cast<int>(k), weights, y,
                                          tab, n, s);
    return launch_status();
}

}  // extern "C"
