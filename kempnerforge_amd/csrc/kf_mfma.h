// MFMA-path helpers shared by the forward, capture and backward kernels.
#pragma once

#include "kf_common.h"

namespace kf {
namespace mfma {

constexpr int BN = 64;     // keys per tile
constexpr int ROWS = 128;  // (query head, position) rows per workgroup

// Physical slot p (0..15) inside a 16-key group of the transposed V holds this
// logical key: lane half h = p/8, slot j = p%8 of the P^T B-operand carries key
// (j<4 ? 4h+j : 8+4h+j-4) because of the 32x32 C layout of S^T.
__device__ __forceinline__ int vt_logical_key(int p) {
  const int h = (p & 15) >> 3, j = p & 7;
  return (p & ~15) + (j < 4 ? 4 * h + j : 8 + 4 * h + (j - 4));
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& u) { return __builtin_bit_cast(bf16x8, u); }

// Block-id remap so that the workgroups one XCD runs are a contiguous range of
// logical ids (the dispatcher deals ids round-robin over the 8 XCDs): blocks of
// one KV head then share that XCD's L2.
__device__ __forceinline__ int xcd_logical_id(int L, int nblk) {
  const int per = nblk / 8, rem = nblk % 8;
  const int xcd = L % 8, idx = L / 8;
  return xcd * per + min(xcd, rem) + idx;
}

struct RowInfo {
  int b, g, hq, pos, p0;
  bool q_valid;
};

__device__ __forceinline__ RowInfo row_info(int logical, int nqb, int Hkv, int n_rep, int bm_pos,
                                            int Sq, int r) {
  RowInfo ri;
  const int bh = logical / nqb;
  const int qb = nqb - 1 - (logical % nqb);  // longest causal rows first
  ri.b = bh / Hkv;
  ri.g = bh % Hkv;
  ri.p0 = qb * bm_pos;
  const bool row_valid = r < n_rep * bm_pos;
  const int hl = row_valid ? r / bm_pos : 0;
  ri.pos = ri.p0 + (row_valid ? r % bm_pos : 0);
  ri.q_valid = row_valid && ri.pos < Sq;
  ri.hq = ri.g * n_rep + hl;
  return ri;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// LDS tiles are stored unpadded, [rows][R] 16-byte chunks, with chunk c of row
// r at position c ^ (r % R): the 32 (or 8, 16) consecutive rows a fragment read
// touches then land in distinct bank groups.  R is 8 or 16.
template <int R>
__device__ __forceinline__ const bf16x8& lds_frag(const bf16* tile, int row, int chunk) {
  return *(const bf16x8*)(tile + (row * R + (chunk ^ (row % R))) * 8);
}

// Copy a [ROWS_T][R chunks] bf16 tile whose rows start `ld` elements apart in
// global memory into a swizzled LDS tile with direct global->LDS loads: each
// instruction moves 64 lanes x 16 bytes into 1 KB of contiguous LDS, so the
// lane picks the global chunk that belongs at its LDS position.  The 4
// wavefronts of the workgroup split the instructions.  Completion is tracked
// by vmcnt: wait with lds_copy_wait() and a barrier before reading the tile.
template <int ROWS_T, int R, int NW = 4>
__device__ __forceinline__ void tile_to_lds(const bf16* __restrict__ g, uint32_t ld, bf16* lds,
                                            int w, int lane) {
  constexpr int TOTAL = ROWS_T * R / 64;
  static_assert(TOTAL % NW == 0, "tile must split evenly over the wavefronts");
  constexpr int PER = TOTAL / NW;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int L = (w * PER + j) * 64 + lane;
    const int row = L / R, pc = L % R;
    const int lc = pc ^ (row % R);
    // uniform base + 32-bit per-lane byte offset: the saddr form of the load
    const uint32_t off = ((uint32_t)row * ld + (uint32_t)lc * 8u) * 2u;
    __builtin_amdgcn_global_load_lds((const void*)((const char*)g + off),
                                     (lds_ptr_t)(lds + (w * PER + j) * 512), 16, 0, 0);
  }
}

// 64 consecutive floats (one per lane of one wavefront) straight into LDS.
__device__ __forceinline__ void row_to_lds(const float* __restrict__ g, float* lds, int lane) {
  __builtin_amdgcn_global_load_lds((const void*)(g + lane), (lds_ptr_t)lds, 4, 0, 0);
}

__device__ __forceinline__ void lds_copy_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wavefront index as a scalar (SGPR) value, so per-wave LDS destinations and
// global bases derived from it stay uniform.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

}  // namespace mfma
}  // namespace kf
