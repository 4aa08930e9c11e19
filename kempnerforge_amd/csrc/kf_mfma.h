// MFMA-path helpers shared by the forward, capture and backward kernels.
#pragma once

#include <climits>

#include "kf_common.h"

namespace kf {
namespace mfma {

constexpr int BN = 64;     // keys per tile
constexpr int ROWS = 128;  // (query head, position) rows per workgroup

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& u) { return __builtin_bit_cast(bf16x8, u); }

// Block-id remap for grids of nblk = nb * G blocks, G per group (the blocks of
// one KV head, numbered longest causal rows first).  The dispatcher deals
// block ids round-robin over the 8 XCDs, each XCD running its share in id
// order.  With nb a multiple of 8, XCD x takes a contiguous range of logical
// ids, whole groups, so the blocks of one KV head share that XCD's L2.  With
// fewer groups a contiguous range would be a group's longest (or shortest)
// blocks, and the XCDs' shares would differ up to threefold: then each group
// is dealt to s = 8 / gcd(nb, 8) XCDs, XCD j of them taking the group's
// blocks j, j + s, j + 2s, ... (still longest first), so the shares balance
// and an XCD still touches few groups.
//
// lane_order(c, n, G) is that deal for a position c of the contiguous
// per-XCD order (used as is by the persistent kernels' shares, xcd_items).
__host__ __device__ __forceinline__ int lane_order(int c, int nblk, int G) {
  const int nb = nblk / G;
  const int s = 8 >> min(__builtin_ctz((unsigned)nb | 8u), 3);  // 8 / gcd(nb, 8)
  if (s == 1) return c;
  // c runs over the groups' lanes in order: lane j of group b holds its blocks
  // j, j + s, ... (q or q + 1 of them, the first m lanes one more)
  const int b = c / G, r = c % G, q = G / s, m = G % s;
  int j, t;
  if (r < m * (q + 1)) {
    j = r / (q + 1);
    t = r % (q + 1);
  } else {
    j = m + (r - m * (q + 1)) / q;
    t = (r - m * (q + 1)) % q;
  }
  return b * G + j + t * s;
}
__host__ __device__ __forceinline__ int xcd_logical_id(int L, int nblk, int G) {
  const int per = nblk / 8, rem = nblk % 8;
  const int xcd = L % 8, idx = L / 8;
  return lane_order(xcd * per + min(xcd, rem) + idx, nblk, G);  // contiguous per XCD, dealt
}

// Persistent schedule over nitems work items: XCD x owns a contiguous range
// of positions (the unmasked kernels pass them through lane_order, as
// xcd_logical_id does for one-item-per-workgroup grids).  With G workgroups per
// XCD (grid = 8G, or grid = nitems for one item each), round r gives the
// workgroup of in-XCD index wi the item r*G + wi of its XCD's range in even
// rounds and r*G + G-1-wi in odd ones: with items ordered longest first, each
// workgroup's rounds pair long items with short ones, so the shares balance.
struct XcdItems {
  int lo, cnt, G, wi;
};
__device__ __forceinline__ XcdItems xcd_items(int nitems) {
  const int per = nitems / 8, rem = nitems % 8, xcd = blockIdx.x % 8;
  return XcdItems{xcd * per + min(xcd, rem), per + (xcd < rem ? 1 : 0),
                  (int)(gridDim.x + 7) / 8, (int)blockIdx.x / 8};
}
// logical item of round r, or -1 when this workgroup is done
__device__ __forceinline__ int xcd_item(const XcdItems& x, int r) {
  const int j = r * x.G + ((r & 1) ? x.G - 1 - x.wi : x.wi);
  return j < x.cnt ? x.lo + j : -1;
}
// Position c of the contiguous per-XCD order (xcd_item) to an item numbered
// group * L + rank (n / L groups of L items, rank 0 the longest), dealt
// longest first over all groups: position j of XCD x is entry 8 j + x of the
// list ordered by (rank, group), so every XCD's share is sorted longest first
// and holds every rank of every group about equally (for grids whose groups
// do not fill the XCDs evenly; the plain contiguous shares keep a group's
// items on one XCD's L2).
__host__ __device__ __forceinline__ int dealt_order(int c, int n, int L) {
  const int per = n / 8, rem = n % 8;
  const int x = c < rem * (per + 1) ? c / (per + 1) : rem + (c - rem * (per + 1)) / per;
  const int i = 8 * (c - x * per - min(x, rem)) + x, ng = n / L;
  return (i % ng) * L + i / ng;
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

// LDS tiles are stored unpadded, [rows][R] 16-byte chunks (R = 8 or 16), with
// chunk c of row r at position c ^ swz<R>(r).  gfx950's LDS has 64 banks of 4
// bytes; ds_read_b128 serves a wavefront in 4 passes of 16 lanes and the 8-byte
// reads (ds_read_b64, ds_read_b64_tr_b16) in 2 passes of 32 lanes, each pass
// 256 bytes wide, and two lanes of a pass that touch different words of one
// bank cost a cycle more.  swz makes every pass of the three read patterns the
// kernels use touch 256 distinct bytes modulo 256:
//  - ds_read_b128, one row per lane, 16 consecutive rows per pass, same chunk:
//    the positions (r % 2, c ^ swz) (R = 8) or c ^ swz (R = 16) must differ;
//  - ds_read_b64_tr_b16 of the backward (lds_frag_t): rows 4k..4k+3 per pass,
//    4 chunks 4j..4j+3 each, so swz >> 2 (R = 16) or bit 2 of swz between rows
//    of one parity (R = 8) must differ;
//  - the decode's transposed V read: rows 8k..8k+7 per pass, chunk pairs
//    2j, 2j+1, so swz >> 1 must differ over the rows (of one parity for R = 8).
// Both forms are bit permutations of row % 16 that satisfy all three
// (measured: 0 bank-conflict cycles per instruction for each pattern, where
// the previous (r % 8, r / 8) interleave cost 4 per ds_read_b128 on 128-byte
// rows and 2 per transposed read on 256-byte rows).
// R = 4 (64-byte rows, only read one row per lane with ds_read_b128): the row's
// 4-row group index, so 16 consecutive rows of one chunk meet 16 distinct
// 16-byte slots of a 256-byte window.
template <int R>
__device__ __forceinline__ int swz(int row) {
  return R == 16  ? (((row & 3) << 2) | ((row >> 1) & 2) | ((row >> 3) & 1))
         : R == 8 ? (((row << 1) & 4) | ((row >> 1) & 2) | ((row >> 3) & 1))
                  : ((row >> 2) & 3);
}

// (E: the tile's 16-bit element type; fragments are bf16x8 containers)
template <int R, typename E>
__device__ __forceinline__ const bf16x8& lds_frag(const E* tile, int row, int chunk) {
  static_assert(sizeof(E) == 2, "16-bit elements");
  return *(const bf16x8*)(tile + (row * R + (chunk ^ swz<R>(row))) * 8);
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Direct global->LDS loads: lane i's bytes land at lds + size * i.  Issued
// from inline asm so that the compiler does not track them: tracked, every
// LDS read behind one waits for all outstanding LDS reads (lgkmcnt(0)) or for
// all of them to land (vmcnt(0)), which serialises software-pipelined LDS
// fragment reads.  Completion is therefore the caller's: an explicit
// s_waitcnt vmcnt (lds_copy_wait) and, across wavefronts, a barrier, before
// the data is read.  `lds` and `base` must be wavefront-uniform.  The LDS
// address goes in m0 as an input operand bound to that register, so the
// compiler itself writes m0 and knows its value (a clobber inside the asm
// would leave any m0 value the compiler keeps live silently overwritten).
//
// KF_VMEM_ASM_NOPS opens every inline-asm memory instruction: the compiler
// cannot see the operands an asm statement reads, so it does not insert the
// wait states the ISA requires between a VALU write of an SGPR (v_readlane,
// v_readfirstlane, e.g. when it reloads a spilled SGPR) and a vector memory
// instruction reading that SGPR as its address base (5), or between an SALU
// write of m0 and an LDS DMA reading it (1).  Without them the load can use
// the stale base and fault.
#define KF_VMEM_ASM_NOPS "s_nop 4\n\t"
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, const void* base) {
  asm volatile(KF_VMEM_ASM_NOPS "global_load_lds_dwordx4 %0, %1"
               : : "v"(voff), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4(uint32_t lds, uint32_t voff, const void* base) {
  asm volatile(KF_VMEM_ASM_NOPS "global_load_lds_dword %0, %1"
               : : "v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// Copy a [ROWS_T][R chunks] 16-bit tile whose rows start `ld` elements apart in
// global memory into a swizzled LDS tile with direct global->LDS loads: each
// instruction moves 64 lanes x 16 bytes into 1 KB of contiguous LDS, so the
// lane picks the global chunk that belongs at its LDS position.  The 4
// wavefronts of the workgroup split the instructions.  Completion is tracked
// by vmcnt: wait with lds_copy_wait() and a barrier before reading the tile.
// Rows at or beyond `rows` (when given) repeat global row rows - 1: a tile
// that runs past the end of an unpadded tensor stays in bounds.
// FRESH: the per-lane offsets are recomputed at every call (a few VALU
// instructions) instead of being kept live across the caller's loop, for
// kernels whose registers are otherwise spent.
template <int ROWS_T, int R, int NW = 4, bool FRESH = false, typename E>
__device__ __forceinline__ void tile_to_lds(const E* __restrict__ g, uint32_t ld, E* lds,
                                            int w, int lane, int rows = ROWS_T) {
  static_assert(sizeof(E) == 2, "16-bit elements");
  constexpr int TOTAL = ROWS_T * R / 64;
  static_assert(TOTAL % NW == 0, "tile must split evenly over the wavefronts");
  constexpr int PER = TOTAL / NW;
  if (FRESH) asm volatile("" : "+v"(lane));
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int L = (w * PER + j) * 64 + lane;
    const int row = L / R, pc = L % R;
    const int lc = pc ^ swz<R>(row);
    // uniform base + 32-bit per-lane byte offset: the saddr form of the load
    const uint32_t off = ((uint32_t)min(row, rows - 1) * ld + (uint32_t)lc * 8u) * 2u;
    dma16(lds_addr(lds + (w * PER + j) * 512), off, g);
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

// Per-lane byte offsets for lds_frag_t on a [rows][D] tile: fragment (c, dt)
// covers rows 16c..16c+15 and columns 32dt..32dt+31.  Rows are 16-aligned, so
// the swizzle term does not depend on c and each lane needs only one
// offset per (dt, first/second read); c adds a compile-time 16-row step
// (swz depends on row % 16 only).
template <int D>
struct TrOffsets {
  uint32_t o[D / 32][2];
};

template <int D>
__device__ __forceinline__ TrOffsets<D> tr_offsets(int lane) {
  constexpr int R = D / 8;
  const int G = lane >> 4, a = lane & 15;
  const int rowA = 4 * (lane >> 5) + (a >> 2), rowB = rowA + 8;
  const int x = 2 * (G & 1) + ((a & 3) >> 1);  // 16-byte chunk inside the 32-column block
  const int within = 4 * (a & 1);              // element inside the chunk
  TrOffsets<D> t;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    const int ch = 4 * dt + x;
    t.o[dt][0] = (uint32_t)(((rowA * R + (ch ^ swz<R>(rowA))) * 8 + within) * 2);
    t.o[dt][1] = (uint32_t)(((rowB * R + (ch ^ swz<R>(rowB))) * 8 + within) * 2);
  }
  return t;
}

// A-operand fragment of a transposed product, read from a row-major swizzled
// [rows][D] LDS tile with two ds_read_b64_tr_b16.
//
// ds_read_b64_tr_b16 works on groups of 16 lanes: address-lane a of a group
// fetches 4 contiguous 16-bit elements, and result-lane i receives element
// (i % 4) of the chunk fetched by address-lane 4e + i/4, for e = 0..3 (the 16
// lanes' 64 elements read as a 4x16 block, one column per lane).  Address-lane
// a = 4e + k of group G therefore fetches row 16c + 4h + e (h = lane / 32),
// columns 32dt + 16 (G % 2) + 4k .. +3, and result-lane l ends up holding column
// 32dt + l % 32 of rows 16c + 4h + e: exactly slots j = 0..3 of the fragment
// whose slot (h, j) carries row 16c + (j < 4 ? 4h + j : 8 + 4h + j - 4).  The
// second read (rows + 8) fills slots 4..7.  That is the slot order of the P^T /
// dS B operands built from the 32x32 C layout, so the products line up.
template <int D, typename E>
__device__ __forceinline__ bf16x8 lds_frag_t(const E* tile, const TrOffsets<D>& t, int c,
                                             int dt) {
  static_assert(sizeof(E) == 2, "16-bit elements");
  const char* base = (const char*)tile + c * 16 * D * 2;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(base + t.o[dt][0]));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(base + t.o[dt][1]));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// 64 consecutive floats (one per lane of one wavefront) straight into LDS.
__device__ __forceinline__ void row_to_lds(const float* __restrict__ g, float* lds, int lane) {
  dma4(lds_addr(lds), (uint32_t)lane * 4u, g);
}

__device__ __forceinline__ void lds_copy_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// s_waitcnt vmcnt(N): all but the last N vector-memory instructions issued
// have completed (gfx950 counts loads, direct-to-LDS loads and stores in one
// counter, in issue order)
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Pin a loaded value at this point: the compiler waits for its load here, not
// at its first use, which may sit inside a loop that keeps direct-to-LDS
// loads in flight (a wait there would stall on those every iteration).
template <typename T>
__device__ __forceinline__ void settle(T& x) {
  asm volatile("" : "+v"(x));
}

// x combined over lanes l and l ^ 32 (the two halves of a 32x32 C column) with
// v_permlane32_swap, a VALU op, instead of __shfl_xor's LDS permute (which
// queues behind the fragment reads).  The swap leaves lanes 0-31 holding
// (x[l], x[l+32]) and lanes 32-63 (x[l-32], x[l]), so max and sum come out as
// max / sum of the pair on both lanes, as with x op __shfl_xor(x, 32).
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wavefront index as a scalar (SGPR) value, so per-wave LDS destinations and
// global bases derived from it stay uniform.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---- packed documents -----------------------------------------------------
// With per-position document ids a query sees a key only inside its own
// document.  kv_prep records each 64-position tile's [min, max] document id;
// a workgroup lists the tiles whose range meets its own range (skipping the
// rest) and applies the element-wise test only to tiles that are not entirely
// in the workgroup's single document.  Min/max ranges make this exact for any
// id pattern, not only contiguous segments.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// explicit-mask kinds of the MFMA kernels (one at a time)
enum { MASK_NONE = 0, MASK_DOC = 1, MASK_KPM = 2 };

constexpr int DOC_MAX_TILES = 4096;      // capacity of a workgroup's tile list
constexpr int DOC_MASK_FLAG = 0x8000;    // list entry: tile needs the element test

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

// Lists, in ascending order, the tiles t in [t0, t1) whose document range
// meets that of rows [p_begin, p_end) (at most 256 rows, p_end > p_begin):
// list[] gets t | DOC_MASK_FLAG, or plain t when the tile and the rows are one
// and the same document.  Returns the count.  Called by one wavefront; the
// caller publishes the count and synchronises before others read the list.
// With list null it only counts.
// The rows' ids and the first 64 tile ranges are loaded together, so the list
// costs one memory round trip for up to 64 tiles.
__device__ __forceinline__ int doc_tile_list(const int32_t* __restrict__ drow, int p_begin,
                                             int p_end, const int2* __restrict__ ranges, int t0,
                                             int t1, uint16_t* list, int lane) {
  int2 r = make_int2(INT_MAX, INT_MIN);
  if (t0 + lane < t1) r = ranges[t0 + lane];
  int lo = INT_MAX, hi = INT_MIN;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int p = p_begin + 64 * j + lane;
    if (p < p_end) {
      const int d = drow[p];
      lo = min(lo, d);
      hi = max(hi, d);
    }
  }
  lo = __builtin_amdgcn_readfirstlane(wave_min_i(lo));
  hi = __builtin_amdgcn_readfirstlane(wave_max_i(hi));
  int n = 0;
  for (int base = t0; base < t1; base += 64) {
    const int t = base + lane;
    if (base != t0) r = t < t1 ? ranges[t] : make_int2(INT_MAX, INT_MIN);
    const bool vis = t < t1 && r.x <= hi && r.y >= lo;
    const bool whole = r.x == r.y && lo == hi && r.x == lo;
    const uint64_t m = __builtin_amdgcn_ballot_w64(vis);
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    if (list != nullptr && vis && n + below < DOC_MAX_TILES)
      list[n + below] = (uint16_t)(t | (whole ? 0 : DOC_MASK_FLAG));
    n += __builtin_popcountll(m);
  }
  return min(n, DOC_MAX_TILES);
}

// ---- key padding ------------------------------------------------------------
// With a key-validity mask (1 = attend) a query sees key j when j <= i and
// key j is valid.  A row that sees no key at all (i before the first valid
// key) is unmasked entirely instead, as the reference's NaN guard does
// (mask | ~mask.any(-1)): it attends every key, future and padded ones
// included.  kv_prep records each 64-key tile's {number of valid keys, first
// valid position or INT_MAX}; the first valid key of the batch row, and with
// it the guarded rows (a prefix), follow from those records.

// First valid key position of the row (INT_MAX if none), from the records of
// tiles [0, ntiles).  Wavefront-uniform.
__device__ __forceinline__ int kpm_first_valid(const int2* __restrict__ rec, int ntiles, int lane) {
  for (int base = 0; base < ntiles; base += 64) {
    const int t = base + lane;
    const int f = __builtin_amdgcn_readfirstlane(wave_min_i(t < ntiles ? rec[t].y : INT_MAX));
    if (f != INT_MAX) return f;
  }
  return INT_MAX;
}

// True when every key of the batch row is valid (tile t holds min(64, S - 64 t)
// valid keys), from the row's tile records; wavefront-uniform.  Such a row is
// plain causal attention: the launches with key padding hand its rows to the
// unmasked kernels.
__device__ __forceinline__ bool kpm_all_valid(const int2* __restrict__ rec, int S, int lane) {
  const int ntiles = (S + BN - 1) / BN;
  bool short_tile = false;
  for (int base = 0; base < ntiles; base += 64) {
    const int t = base + lane;
    if (t < ntiles) short_tile |= rec[t].x != min(BN, S - BN * t);
  }
  return __builtin_amdgcn_ballot_w64(short_tile) == 0;
}

// Lists, in ascending order, tiles t in [t0, t1) for which pick(t, rec[t])
// returns nonzero (2: with DOC_MASK_FLAG).  Same contract as doc_tile_list.
template <typename Pick>
__device__ __forceinline__ int kpm_tile_list(const int2* __restrict__ rec, int t0, int t1,
                                             Pick pick, uint16_t* list, int lane) {
  int n = 0;
  for (int base = t0; base < t1; base += 64) {
    const int t = base + lane;
    const int sel = t < t1 ? pick(t, rec[t]) : 0;
    const uint64_t m = __builtin_amdgcn_ballot_w64(sel != 0);
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    if (sel && n + below < DOC_MAX_TILES)
      list[n + below] = (uint16_t)(t | (sel == 2 ? DOC_MASK_FLAG : 0));
    n += __builtin_popcountll(m);
  }
  return min(n, DOC_MAX_TILES);
}

}  // namespace mfma
}  // namespace kf
