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

}  // namespace mfma
}  // namespace kf
