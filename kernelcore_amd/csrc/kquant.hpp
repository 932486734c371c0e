// kquant.hpp -- device-side definitions shared by the K-quant kernels (HIP, gfx950).
//
// Weight stream layout (this device's; the reference's CPU stream is an 8-row word interleave,
// llm/llm_reference.cpp:385-411). Rows are grouped in tiles of kTileRows = 16 and super-blocks
// (256 weights) in groups of kGroupSb = 4. For tile t and group g, the 64 (super-block, row)
// pairs form the 64 lanes of one wavefront: lane = kq * 16 + r covers row 16t + r, super-block
// 4g + kq. Their ggml blocks are cut into 16-byte pieces and stored piece-major ("slabs" of
// 64 x 16 B = 1 KiB), so that one dwordx4 load per lane reads a whole slab contiguously:
//   Q4_K: 9 slabs = bytes 0..143 of block_q4_K (d, dmin, scales[12] | qs[128]).
//   Q6_K: 13 slabs = bytes 0..207 of block_q6_K (ql[128] | qh[64] | scales[16]), then the 64
//         fp16 d values (128 B).
// Segment (t, g) starts at (t * ngroups + g) * seg_bytes. Rows past `rows` and super-blocks past
// nsb are zero. Apart from that padding the stream holds exactly the ggml bytes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace kcamd {

constexpr int kTileRows = 16;
constexpr int kGroupSb = 4;
constexpr int kQ4kBlock = 144;
constexpr int kQ6kBlock = 210;
constexpr int kQ4kSlabs = 9;
constexpr int kQ6kSlabs = 13;
constexpr int kQ4kSeg = kQ4kSlabs * 1024;       // 9216 B
constexpr int kQ6kSeg = kQ6kSlabs * 1024 + 128;  // 13440 B

inline int tilesOf(int rows) { return (rows + kTileRows - 1) / kTileRows; }
inline int groupsOf(int nsb) { return (nsb + kGroupSb - 1) / kGroupSb; }
inline size_t streamBytes(int qtype_is_q6k, int rows, int k) {
    return size_t(tilesOf(rows)) * size_t(groupsOf(k / 256)) * size_t(qtype_is_q6k ? kQ6kSeg : kQ4kSeg);
}

}  // namespace kcamd
