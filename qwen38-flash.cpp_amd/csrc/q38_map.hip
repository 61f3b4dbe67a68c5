// q38_map.hip — the decoder's optional MLP output map (DecoderLayer::apply_mlp_output_map,
// src/decoder_layer.cpp:198-210; tensors mlp.T, or the low-rank pair mlp.T_delta_left /
// mlp.T_delta_right, :158-182): with the full map out = T(y . T); with the low-rank pair
// t = T(y . L), out = T(y + T(t . R)). y, the maps and the results are bf16.
//
// Each product [rows, K] x [K, N] runs as two launches with a fixed summation order:
//   k_map_part    per (64 columns, 128-input slice): one thread per column n, the slice's
//                 inputs in ascending order with fmaf in float for every row (the rows'
//                 inputs staged in LDS as float, the map's row k read 128 bytes at a time
//                 across the columns); one float partial per (slice, row, column);
//   k_map_finish  per (row, column): the slices' partials added in slice order, rounded to
//                 bf16, plus the residual (the low-rank form's y) and rounded again.
#include "q38_device.hpp"
#include "q38_internal.hpp"

namespace q38 {

namespace {

constexpr int kMapCols = 64;    // columns per workgroup
constexpr int kMapSlice = 128;  // inputs per slice
constexpr int kMapRows = 16;    // rows per call

__global__ __launch_bounds__(kMapCols) void k_map_part(const uint16_t* __restrict__ a, int rows, int K,
                                                       const uint16_t* __restrict__ W, int N, float* __restrict__ part) {
    __shared__ float as[kMapRows][kMapSlice];
    const int tid = threadIdx.x, n = blockIdx.x * kMapCols + tid, s = blockIdx.y, k0 = s * kMapSlice;
    const int nk = K - k0 < kMapSlice ? K - k0 : kMapSlice;
    for (int i = tid; i < rows * nk; i += kMapCols) {
        const int r = i / nk, k = i % nk;
        as[r][k] = bf2f(a[static_cast<size_t>(r) * K + k0 + k]);
    }
    __syncthreads();
    if (n >= N) return;
    float acc[kMapRows];
#pragma unroll
    for (int r = 0; r < kMapRows; ++r) acc[r] = 0.0f;
    const uint16_t* wc = W + static_cast<size_t>(k0) * N + n;
#pragma unroll 8
    for (int k = 0; k < nk; ++k) {
        const float wv = bf2f(wc[static_cast<size_t>(k) * N]);
#pragma unroll
        for (int r = 0; r < kMapRows; ++r)
            if (r < rows) acc[r] = fmaf(as[r][k], wv, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < kMapRows; ++r)
        if (r < rows) part[(static_cast<size_t>(s) * rows + r) * N + n] = acc[r];
}

__global__ __launch_bounds__(256) void k_map_finish(const float* __restrict__ part, int ns, int rows, int N,
                                                    const uint16_t* __restrict__ resid, uint16_t* __restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * N) return;
    const int r = i / N, n = i % N;
    float sum = 0.0f;
    for (int s = 0; s < ns; ++s) sum += part[(static_cast<size_t>(s) * rows + r) * N + n];
    const float v = bf2f(f2bf(sum));
    out[i] = resid ? f2bf(bf2f(resid[i]) + v) : f2bf(v);
}

// out [rows, N] = T(a [rows, K] . W [K, N]) (+ resid, rounded); part: K / 128 x rows x N floats.
hipError_t map_product(const uint16_t* a, int rows, int K, const uint16_t* W, int N, const uint16_t* resid,
                       uint16_t* out, float* part, hipStream_t st) {
    const int ns = (K + kMapSlice - 1) / kMapSlice;
    hipError_t e = launch(k_map_part, dim3((N + kMapCols - 1) / kMapCols, ns), dim3(kMapCols), 0, st, a, rows, K, W,
                          N, part);
    if (e != hipSuccess) return e;
    return launch(k_map_finish, dim3((rows * N + 255) / 256), dim3(256), 0, st, static_cast<const float*>(part), ns,
                  rows, N, resid, out);
}

size_t round256(size_t v) { return (v + 255) / 256 * 256; }

} // namespace

size_t mlp_map_workspace(int hidden, int rank, int rows) {
    const size_t H = static_cast<size_t>(hidden), R = static_cast<size_t>(rank > 0 ? rank : hidden);
    const size_t ns = (H + kMapSlice - 1) / kMapSlice;
    // the partials of the widest product, then the low-rank intermediate t [rows, rank]
    return round256(ns * static_cast<size_t>(rows) * H * 4) + round256(static_cast<size_t>(rows) * R * 2);
}

hipError_t launch_mlp_map(const MlpMapDev& m, const uint16_t* y, int rows, uint16_t* out, void* ws, hipStream_t st) {
    if (rows < 1 || rows > kMapRows) return hipErrorInvalidValue;
    const size_t H = static_cast<size_t>(m.hidden);
    float* part = static_cast<float*>(ws);
    uint16_t* t = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) +
                                              round256(((H + kMapSlice - 1) / kMapSlice) * rows * H * 4));
    if (m.rank == 0) return map_product(y, rows, m.hidden, m.full, m.hidden, nullptr, out, part, st);
    hipError_t e = map_product(y, rows, m.hidden, m.left, m.rank, nullptr, t, part, st);
    if (e != hipSuccess) return e;
    return map_product(t, rows, m.rank, m.right, m.hidden, y, out, part, st);
}

} // namespace q38
