// launch.hpp -- host-side launchers of the HIP kernels, called by the built-in kernel table
// (llm_kernels.cpp) after argument validation. Each returns a kc error code (0 = success) and
// only enqueues work on `s`.
#pragma once

#include <hip/hip_runtime.h>
#include <kernelcore/llm_kernels.h>

namespace kcamd {

// The MFMA matmul's activation operands of a batch of ncols per-256-quantized columns of length k,
// as a quantizer can write them next to the slots: the int8 values x as fp16 16 x act[ncols][k], the
// Q4_K min operands mins[ncols][k / 256][16] (fp16: 64 (B_j >> 6) for the 8 sums B_j of 32, then
// B_j & 63) and the scales xdT[k / 256][ncp], ncp = ncols rounded up to 128.
struct ActF16 {
    void* act;
    void* mins;
    float* xdT;
    int ncp;
};
inline int actF16Cols(int ncols) { return (ncols + 127) / 128 * 128; }
// Bytes of an ActF16 buffer for up to max_cols columns (act, then mins, then xdT).
inline size_t actF16Bytes(int max_cols, int k) {
    return (size_t)max_cols * k * 2 + (size_t)max_cols * (k / 256) * 32 + (size_t)(k / 256) * actF16Cols(max_cols) * 4;
}
// The ActF16 view of such a buffer for ncols columns.
inline ActF16 actF16View(void* base, int max_cols, int k, int ncols) {
    char* b = static_cast<char*>(base);
    return ActF16{b, b + (size_t)max_cols * k * 2, reinterpret_cast<float*>(b + (size_t)max_cols * k * 2 + (size_t)max_cols * (k / 256) * 32),
                  actF16Cols(ncols)};
}


// kquant.hip
int launchRepack(const kcKquantRepackArgs& a, bool unpack, hipStream_t s);
int launchQuantizeQ8x4(const float* x, int* xq, float* xd, int count, hipStream_t s);
int launchQuantizeCols(const float* x, int* q, int k, int ncols, hipStream_t s);
int launchQuantizeColsK(const float* x, int* q, int k, int ncols, hipStream_t s, const ActF16* ao = nullptr);
int launchMatvecKq(bool q6k, const kcMatvecQ4Q8Args& a, hipStream_t s);
// kmatmul.hip: column-tiled matmul (any ncols; bit-identical per column to the reference).
int launchMatmulCols(bool q6k, bool per256, const kcMatmulKQ8Args& a, hipStream_t s);
// kmatmul_mfma.hip: K-quant x per-256 activations on MFMA (large batches).
int launchMatmulMfma(bool q6k, const kcMatmulKQ8Args& a, hipStream_t s);
// The per-stream scratch a by-name per-256 matmul of these sizes stages its fp16 activations (and
// K-split partial sums) in; 0 when it takes a path without it.
size_t matmulStagingBytes(int rows, int k, int ncols);
// The matmul names: column tiles for small batches and per-32 slots, MFMA for large per-256 batches.
int launchMatmulKq(bool q6k, bool per256, const kcMatmulKQ8Args& a, hipStream_t s);
// The same kernels with the MFMA activations staged in the fixed device array (kcLaunchMatmulNoAlloc):
// no allocation; InvalidValue when the staging exceeds fixedScratchBytes().
int launchMatmulKqNoAlloc(bool q6k, bool per256, const kcMatmulKQ8Args& a, hipStream_t s);
// Looks up this device's address of the fixed array (once per device, with the device current).
int fixedScratchInit(int device);
size_t fixedScratchBytes();
// One weight matrix of a grouped matmul: y[z] receives the partial sums of K range z.
struct MmPart {
    const void* qw;  // device stream of kcamd::streamBytes layout
    float* y[2];
    int rows;
    int q6;  // Q6_K (else Q4_K)
};
// Whether launchMatmulGroup with part_ks splits the Q6_K parts (those given a y[1]) of this group of
// parts over K (their workgroups then end with the Q4_K parts').
bool matmulGroupSplitsQ6(const MmPart* parts, int nparts, int k, int ncols);
// parts[0..nparts) (at most 3) times the same per-256 activations (ncols columns of length k) in
// one launch where the MFMA kernel applies, K split into ks <= 2 ranges: *used_ks = the split
// taken (1: each y[0] holds the whole product; 2: y[0] + y[1] is the product).
// pre (may be null): the activations already in the MFMA layout (then no conversion is launched).
// part_ks (may be null): each part's own split, reported per part; with it, a Q6_K part that has a
// y[1] may take two K ranges in a group of one (its partial sums y[0] + y[1]), the others one.
int launchMatmulGroup(const MmPart* parts, int nparts, const int* xq, int k, int ncols, int ks, int* used_ks,
                      hipStream_t s, const ActF16* pre = nullptr, int* part_ks = nullptr);
// Whether a group of ncols >= 64 columns of k values runs on the fp16-activation MFMA kernel.
bool mfmaHUsable(int ncols, int k);
// launchMatmulGroup given the MFMA layout (pre) reads only that layout, never the int8 slots xq
bool matmulGroupReadsActOnly(int ncols, int k);
// The K ranges a launch of this shape and weight type takes (2 where one K range would leave compute
// units idle).
int matmulKs(int rows, int k, int ncols, bool q6);
// kmatmul_f16.hip: Y [ncols][rows] = W X, W row-major fp16 [rows][k], x ncols columns of k floats;
// rows % 8 == 0, k even.
int launchMatmulF16(const void* w, const float* x, float* y, int rows, int k, int ncols, hipStream_t s);
// layer_ops.hip
int launchVectorAdd(const float* a, const float* b, float* out, int count, hipStream_t s);
// out = a + (b + b2) (b2 may be null: out = a + b; a null: the sums of squares of b (+ b2) only).
int launchAddSumsq(const float* a, const float* b, float* out, int* q, int n, int rows, hipStream_t s,
                   const float* b2 = nullptr);
int launchNormMulQ8(bool per256, const kcNormMulQ8Args& a, hipStream_t s);
// add_sumsq_f (a, b given) or sumsq_part, then norm_mul_q8_f, in one workgroup per row (n <= 8192).
int launchAddNormQ8(const float* a, const float* b, float* x, const float* w, float* y, int* q, int n, int rows,
                    float eps, hipStream_t s);
// Batch fusions of the model path: x = a + (b [+ b2]) into out (a null: x = b), RMS norm with w
// and per-256 quantization into q (rows slots of n / 256 * 85 ints); RoPE of q into qr and of k,
// with k and v (+ v2, when given) stored as fp16 into cache rows pos[t] (dst_row 32-bit words per
// row).
// (ao, when given, also receives the MFMA layout of the quantized rows; y, when given, the normed
// rows x r w in f32, the values that are quantized.)
int launchAddNormQ8K(const float* a, const float* b, const float* b2, float* out, const float* w, int* q, int n,
                     int rows, float eps, hipStream_t s, const ActF16* ao = nullptr, float* y = nullptr);
int launchSiluMulQ8KAct(const kcSiluMulQ8FArgs& a, const ActF16* ao, hipStream_t s);
int launchRopeQKStore(const float* q, float* qr, const float* k, const float* v, int* kcache, int* vcache,
                      const int* pos, const float* ff, int head_dim, int nh, int nkv, int n, float log2_base, int neox,
                      int dst_row, int dst_rows, hipStream_t s, const float* v2 = nullptr);
// The same with the per-head q / k norms first (x r w with the weights qw / kw, eps): RMS_NORM +
// MUL of each head row of q and of k in the same launch (head_dim 64 or 128, q and k 16-byte
// aligned), the same floats as launchRmsNorm before launchRopeQKStore.
int launchNormRopeQKStore(const float* q, float* qr, const float* k, const float* v, const float* qw, const float* kw,
                          int* kcache, int* vcache, const int* pos, const float* ff, int head_dim, int nh, int nkv,
                          int n, float log2_base, int neox, int dst_row, int dst_rows, float eps, hipStream_t s,
                          const float* v2 = nullptr);
int launchSiluMulQ8(bool per256, const kcSiluMulQ8FArgs& a, hipStream_t s);
int launchMulRows(const kcMulRowsArgs& a, hipStream_t s);
int launchSiluMul(const kcSiluMulArgs& a, hipStream_t s);
int launchRmsNorm(const kcRmsNormArgs& a, hipStream_t s);
int launchRope(const kcRopeGgmlArgs& a, hipStream_t s);
// ROPE of q and k, and the fp16 rows of the roped k and of v into the caches at rows idx (int64),
// in one launch; the roped k also kept in kr (layer_ops.hip rope_kv_rows_kernel).
struct RopeKvRows {
    const float* q;
    float* qr;
    const float* k;
    float* kr;
    const float* v;
    int *kcache, *vcache;
    const int* pos;
    const int* idx;
    const float* ff;
    int head_dim, nh, nkv, n;
    float log2_base;
    bool neox;
    int src_v, k_row, v_row, dst_rows;  // v row stride (floats), cache row strides (32-bit words), cache rows
    const float* v2;                    // may be null: v's product in two K ranges, v + v2 stored (and into v)
};
int launchRopeKvRows(const RopeKvRows& r, hipStream_t s);
int launchSetRows(const kcSetRowsF16Args& a, hipStream_t s);
int launchFaScores(const kcFaScoresArgs& a, hipStream_t s);
int launchFaMax(const kcFaMaxArgs& a, hipStream_t s);
int launchFaExp(const kcFaExpArgs& a, hipStream_t s);
int launchFaValues(const kcFaValuesArgs& a, hipStream_t s);
int launchFlashAttn(const kcFlashAttnArgs& a, hipStream_t s);
constexpr int kFlashAttnMaxT = 16384;
// Largest k the matvec's activation staging accepts.
constexpr int kMatvecMaxK = 32768;

}  // namespace kcamd
