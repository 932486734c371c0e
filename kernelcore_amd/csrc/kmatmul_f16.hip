// kmatmul_f16.hip -- Y = W X for fp16 weights and fp32 activations (gfx950): the matmul_f16 name
// (reference kernels/llm/matmul_f16.cu, mirror llm/llm_reference.cpp:756-764 in
// arasheedu/Kernelcore; the ggml backend sends F16 weights there with the activations as they are,
// integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:559-566).
//
// The weights stay in ggml's row-major F16 layout (W[r][k], two values per 32-bit word): a
// wavefront reads whole rows with 16-byte loads, so no load-time interleave is needed (the
// reference's 8-row word interleave, llm_reference.cpp:740-746, serves 8 CPU vector lanes).
// Three kernels, by batch width:
//   * ncols <= 8 (decode): one wavefront per 2 rows; each lane multiplies 8 consecutive values of
//     a row with the same 8 values of every column, the partial sums are reduced across the 64
//     lanes. HBM-bound (2 bytes per weight).
//   * ncols > 8: v_mfma_f32_32x32x16_f16 on 32 x 32 output tiles, four per workgroup. The weights
//     are exact fp16 operands; each activation is split into hi = fp16(x) and lo = fp16(x - hi)
//     and every product runs as two MFMAs (f32 accumulation), within about 2^-22 of the fp32
//     product (a single fp16 rounding of x would be 2^-11).
//   * k not a multiple of 8 (the reference allows any even k): one thread per output, the
//     reference's own loop.
// Sums run in a different order than the reference's sequential loop (a tree over the lanes, the
// MFMA's accumulation): within the 1e-3 relative bar, not bit-identical.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.hpp"
#include "launch.hpp"

namespace kcamd {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits); }

// Sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float waveSum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---- ncols <= 8: two rows per wavefront, NC columns (the launcher rounds ncols up to 1, 2, 4
// or 8; surplus columns reread the last one and are not stored). k % 8 == 0.
template <int NC>
__global__ __launch_bounds__(256) void mmf16_vec_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                        float* __restrict__ y, int rows, int k, int ncols) {
    constexpr int R = 2;
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * R;
    if (r0 >= rows) return;  // rows % 8 == 0: a live wavefront has both rows
    const int nch = k / 8;   // 16-byte chunks per row
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    for (int ch = lane; ch < nch; ch += 64) {
        u32x4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + (size_t)(r0 + r) * k) + ch);
        float4 xv[NC][2];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float4* xp = reinterpret_cast<const float4*>(x + (size_t)min(c, ncols - 1) * k) + 2 * ch;
            xv[c][0] = xp[0];
            xv[c][1] = xp[1];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float wf[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wf[2 * e] = h2f(wv[r][e] & 0xFFFFu);
                wf[2 * e + 1] = h2f(wv[r][e] >> 16);
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float xs[8] = {xv[c][0].x, xv[c][0].y, xv[c][0].z, xv[c][0].w,
                                     xv[c][1].x, xv[c][1].y, xv[c][1].z, xv[c][1].w};
                float s = acc[r][c];
#pragma unroll
                for (int e = 0; e < 8; ++e) s += wf[e] * xs[e];
                acc[r][c] = s;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float t = waveSum(acc[r][c]);
            if (lane == 0 && c < ncols) y[(size_t)c * rows + r0 + r] = t;
        }
}

// ---- ncols > 8, k % 16 == 0: a workgroup of 4 wavefronts covers 64 rows x 64 columns, each
// wavefront one 32 x 32 tile. Lane (j, h) (j = lane % 32, h = lane / 32) holds, per K-step of 16,
// A = W[row0 + j][k0 + 8h .. +8] and B = x[col0 + j][k0 + 8h .. +8]; the accumulator's register
// v holds output row 8 (v / 4) + 4 h + v % 4 of column j. Rows and columns past the end reread
// the last ones and are not stored.
__global__ __launch_bounds__(256) void mmf16_mfma_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                         float* __restrict__ y, int rows, int k, int ncols) {
    constexpr int U = 4;  // K-steps whose loads are issued together
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
    const int row0 = blockIdx.x * 64 + (wave & 1) * 32, col0 = blockIdx.y * 64 + (wave >> 1) * 32;
    if (row0 >= rows || col0 >= ncols) return;
    const uint16_t* wr = w + (size_t)min(row0 + j, rows - 1) * k + 8 * h;
    const float* xr = x + (size_t)min(col0 + j, ncols - 1) * k + 8 * h;
    f32x16 acc = {};
    const int steps = k / 16;
    int st = 0;
    for (; st + U <= steps; st += U) {
        h8 a[U];
        float4 xv[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            a[u] = __builtin_nontemporal_load(reinterpret_cast<const h8*>(wr + 16 * (st + u)));
            const float4* xp = reinterpret_cast<const float4*>(xr + 16 * (st + u));
            xv[u][0] = xp[0];
            xv[u][1] = xp[1];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float xs[8] = {xv[u][0].x, xv[u][0].y, xv[u][0].z, xv[u][0].w,
                                 xv[u][1].x, xv[u][1].y, xv[u][1].z, xv[u][1].w};
            h8 bh, bl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 hi = (_Float16)xs[e];
                bh[e] = hi;
                bl[e] = (_Float16)(xs[e] - (float)hi);
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[u], bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[u], bl, acc, 0, 0, 0);
        }
    }
    for (; st < steps; ++st) {
        const h8 a = *reinterpret_cast<const h8*>(wr + 16 * st);
        const float4* xp = reinterpret_cast<const float4*>(xr + 16 * st);
        const float4 x0 = xp[0], x1 = xp[1];
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        h8 bh, bl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const _Float16 hi = (_Float16)xs[e];
            bh[e] = hi;
            bl[e] = (_Float16)(xs[e] - (float)hi);
        }
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, acc, 0, 0, 0);
    }
    const int col = col0 + j;
    if (col >= ncols) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = row0 + 8 * (v / 4) + 4 * h + (v % 4);
        if (row < rows) y[(size_t)col * rows + row] = acc[v];
    }
}

// ---- any even k: one thread per (row, column), the reference's loop (llm_reference.cpp:756-764).
__global__ __launch_bounds__(256) void mmf16_simple_kernel(const uint32_t* __restrict__ w, const float* __restrict__ x,
                                                           float* __restrict__ y, int rows, int k, int ncols) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)rows * ncols) return;
    const int c = (int)(idx / rows), r = (int)(idx % rows);
    const uint32_t* wr = w + (size_t)r * (k / 2);
    const float* xc = x + (size_t)c * k;
    float a = 0.0f;
    for (int i = 0; i < k / 2; ++i) {
        const uint32_t q = wr[i];
        a += h2f(q & 0xFFFFu) * xc[2 * i] + h2f(q >> 16) * xc[2 * i + 1];
    }
    y[(size_t)c * rows + r] = a;
}

}  // namespace

int launchMatmulF16(const void* w, const float* x, float* y, int rows, int k, int ncols, hipStream_t s) {
    if (rows <= 0 || rows % 8 || k <= 0 || k % 2 || ncols <= 0)
        return fromHip(hipErrorInvalidValue, "matmul_f16: shape");
    const uint16_t* wh = static_cast<const uint16_t*>(w);
    // the vector kernels read 16 bytes at a time: w and x 16-byte aligned (hipMalloc gives 256)
    const bool a16 = ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15) == 0;
    if (a16 && k % 8 == 0 && (ncols <= 8 || k % 16)) {
        // columns in launches of at most 8 (only when k % 16 != 0 rules out the MFMA kernel)
        for (int c0 = 0; c0 < ncols; c0 += 8) {
            const int nc = ncols - c0 < 8 ? ncols - c0 : 8;
            const dim3 grid((rows / 2 + 3) / 4), block(256);
            const float* xc = x + (size_t)c0 * k;
            float* yc = y + (size_t)c0 * rows;
            if (nc == 1) hipLaunchKernelGGL(mmf16_vec_kernel<1>, grid, block, 0, s, wh, xc, yc, rows, k, nc);
            else if (nc == 2) hipLaunchKernelGGL(mmf16_vec_kernel<2>, grid, block, 0, s, wh, xc, yc, rows, k, nc);
            else if (nc <= 4) hipLaunchKernelGGL(mmf16_vec_kernel<4>, grid, block, 0, s, wh, xc, yc, rows, k, nc);
            else hipLaunchKernelGGL(mmf16_vec_kernel<8>, grid, block, 0, s, wh, xc, yc, rows, k, nc);
        }
    } else if (a16 && k % 16 == 0) {
        const dim3 grid((rows + 63) / 64, (ncols + 63) / 64), block(256);
        hipLaunchKernelGGL(mmf16_mfma_kernel, grid, block, 0, s, wh, x, y, rows, k, ncols);
    } else {
        const long long n = (long long)rows * ncols;
        hipLaunchKernelGGL(mmf16_simple_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           static_cast<const uint32_t*>(w), x, y, rows, k, ncols);
    }
    return fromHip(hipGetLastError(), "matmul_f16");
}

}  // namespace kcamd
