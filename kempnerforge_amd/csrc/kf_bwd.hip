// bf16 / fp16 MFMA backward attention for gfx950 (head_dim 64 or 128).
//
// Four launches, no atomics (bit-deterministic):
//  kv_prep      (shared with the forward) per KV head: K rotated (eager
//               RoPE) [bh][P][D], rows past S zero.
//  q_prep_bwd   per query head: Q rotated [bhq][P][D]; lse*log2(e) and Delta =
//               rowsum(dO o O) [bhq][P].  P = S rounded up to 128; padded rows
//               are zero with lse = +inf, so they contribute nothing.  dO and V
//               are read in place ([B, S, H, D]) by the kernels below, rows past
//               S repeating row S - 1 (or zero).
//  Transposed operands (K^T, Q^T, dO^T) are never stored: they are read from
//  the row-major LDS tiles with ds_read_b64_tr_b16 (lds_frag_t).
//  dkdv         workgroup = 128 keys of one KV head (4 wavefronts x 32 keys,
//               K and V held in registers as MFMA B operands), looping over every
//               query head of the group and every query tile of 64: the
//               repeat_interleave backward (sum over the group) happens in the
//               accumulators.  S = Q K^T and dP = dO V^T land in the 32x32 C
//               layout with one key per lane; P and dS then feed dV^T += dO^T P
//               and dK^T += Q^T dS as B operands directly.  RoPE backward and the
//               softmax scale are applied at the dK store.  When the caller's
//               workspace holds them it also writes every dS tile (16-bit) to a
//               record for dQ (with key padding: for the batch rows whose first
//               key is valid).
//  dq_ds        (dS records kept) dQ^T += K^T dS^T from the records: one
//               product per element and one read of the dS bytes, HBM-bound.
//               With key padding it serves the batch rows whose first key is
//               valid and dq the others.
//  dq           (otherwise) forward-shaped: 256 (head, position) rows per
//               workgroup sharing each K/V tile; recomputes S^T = K Q^T and
//               dP^T = V dO^T, then dQ^T += K^T dS^T.
//               Both apply RoPE backward at the dQ store.
//  Without an explicit mask dkdv and dq run persistent, one workgroup per CU
//  walking its XCD's items in the zigzag order of xcd_item (long causal items
//  paired with short ones).
// The algorithm is the standard flash-attention backward (recompute P from the
// saved log-sum-exp; dS = P o (dP - Delta)).
//
// Packed documents (MASK_DOC): kv_prep records each 64-position tile's
// document-id range.  dkdv walks only the query tiles whose range meets its key
// block's, dq only the key tiles whose range meets its rows'; tiles not
// entirely in the workgroup's single document get P = 0 where doc[query] !=
// doc[key].  Key padding (MASK_KPM): kv_prep records each tile's valid-key
// count and first valid key; tiles without a valid key are skipped, rows before
// the batch row's first valid key (guarded) see every key, the others need
// the key valid.
#include "kf_common.h"
#include "kf_internal.h"
#include "kf_mfma.h"

#include <algorithm>
#include <type_traits>

namespace kf {

namespace {

using namespace mfma;

constexpr int BKV = 128;  // keys per dK/dV workgroup
constexpr int BQ = 64;    // queries per dK/dV tile

__host__ __device__ constexpr int pad_len(int S) { return (S + BKV - 1) / BKV * BKV; }

// dS records.  The dK/dV kernel writes every dS tile it computes, in the
// input's 16-bit type, for
// the dQ kernel to read instead of recomputing S and dP (with key padding only
// for batch rows without guarded rows, i.e. whose key 0 is valid: a guarded
// row sees keys past the diagonal, outside this layout).
// A record is one dS wavefront's tile: DSQ query positions x DSK keys of one
// query head, 4 KB, stored as that wavefront's four MFMA B operands exactly as
// they sit in registers: [chunk c][lane][8 elements], lane = 32*hh + key, slot
// 4*half + j = row 16c + 8*half + 4*hh + j.  Records are ordered (KV head,
// query tile, key column, query head of the group); with a causal mask only
// the key columns k32 <= 2*qt + 1 that the tile's rows can see exist.
constexpr int DSQ = DS_REC_Q;  // query positions per record (= BQ)
constexpr int DSK = DS_REC_K;  // keys per record (one dS wavefront)
static_assert(DSQ == BQ, "one record row block per query tile");
constexpr int DS_DOC_MAX_TILES = 1024;  // explicit masks keep records up to S = 65536

// record pair index of (KV head bh, query tile qt, key column k32); nqtp = P / DSQ
__host__ __device__ inline int64_t ds_pair(int bh, int qt, int k32, int nqtp, int causal) {
  return causal ? (int64_t)bh * nqtp * (nqtp + 1) + (int64_t)qt * (qt + 1) + k32
                : ((int64_t)bh * nqtp + qt) * (2 * nqtp) + k32;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void q_prep_bwd_kernel(
    const T* __restrict__ q, const T* __restrict__ out, const T* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ cos, const float* __restrict__ sin,
    T* __restrict__ qrot, float* __restrict__ lse2, float* __restrict__ delta, int S, int P,
    int Hq, float inv_scale) {
  constexpr int HALF = D / 2, CP = HALF / 8, TPR = D / 8;
  const int s0 = blockIdx.x * BN, bhq = blockIdx.y, b = bhq / Hq, h = bhq % Hq;
  const int tid = threadIdx.x;
  // q null: the rotated rows are already in qrot (written by the forward)
  for (int it = tid; q != nullptr && it < BN * CP; it += 256) {
    const int row = it / CP, c = it % CP, s = s0 + row;
    u32x4 o1 = {0u, 0u, 0u, 0u}, o2 = {0u, 0u, 0u, 0u};
    if (s < S) {
      // q and O are read once here: non-temporal loads (streaming, ~15% faster
      // from HBM than cached ones); dO stays cached for the kernels after
      const T* src = q + (((int64_t)b * S + s) * Hq + h) * D;
      float x1[8], x2[8];
      unpack8<T>(__builtin_nontemporal_load((const u32x4*)(src + 8 * c)), x1);
      unpack8<T>(__builtin_nontemporal_load((const u32x4*)(src + 8 * c + HALF)), x2);
      rope8<T>(x1, x2, cos + (int64_t)s * HALF + 8 * c, sin + (int64_t)s * HALF + 8 * c, o1,
                 o2);
    }
    T* dst = qrot + ((int64_t)bhq * P + s) * D;
    *(u32x4*)(dst + 8 * c) = o1;
    *(u32x4*)(dst + 8 * c + HALF) = o2;
  }
  // -Delta (TPR consecutive lanes own one row; stored negated so that the dK/dV
  // kernel can start its dP accumulation from it); dO itself is read in place
  // by the dK/dV and dQ kernels
  // all of a thread's dO and O loads are issued before the first reduction
  constexpr int NIT = BN * TPR / 256;
  u32x4 ad[NIT], ao[NIT];
#pragma unroll
  for (int k = 0; k < NIT; ++k) {
    const int it = tid + 256 * k;
    const int row = it / TPR, c = it % TPR, s = s0 + row;
    const int64_t off = (((int64_t)b * S + min(s, S - 1)) * Hq + h) * D + 8 * c;
    ad[k] = *(const u32x4*)(dout + off);
    ao[k] = __builtin_nontemporal_load((const u32x4*)(out + off));
  }
#pragma unroll
  for (int k = 0; k < NIT; ++k) {
    const int it = tid + 256 * k;
    const int row = it / TPR, c = it % TPR, s = s0 + row;
    float part = 0.f;
    if (s < S) {
      float fd[8], fo[8];
      unpack8<T>(ad[k], fd);
      unpack8<T>(ao[k], fo);
#pragma unroll
      for (int j = 0; j < 8; ++j) part += fd[j] * fo[j];
    }
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) part += __shfl_xor(part, o, 64);
    if (c == 0) {
      delta[(int64_t)bhq * P + s] = -part;
      // -lse / scale: the dK/dV kernel starts its S accumulation from it, so
      // that P = exp2(scale log2(e) x) (rows past S: -inf, P = 0)
      lse2[(int64_t)bhq * P + s] = s < S ? -lse[(int64_t)bhq * S + s] * inv_scale : -INFINITY;
    }
  }
}

// dK/dV workgroup: 8 wavefronts on the same 128 keys, two roles that split the
// four products evenly.  Wavefronts 0-3 ("P waves") compute S = Q K^T, turn it
// into P (16-bit) and accumulate dV^T += dO^T P; they hand P to the wavefront of
// the other role that owns the same 32 keys through LDS.  Wavefronts 4-7
// ("dS waves") compute dP = dO V^T meanwhile, then dS = P o (dP - Delta) and
// accumulate dK^T += Q^T dS.  Each role needs only its own B operands and
// accumulators, so two wavefronts fit per SIMD and overlap each other.
template <typename T, int D>
struct DkdvStage {
  T q[BQ * D], o[BQ * D];
  float l[BQ], dl[BQ];  // -lse / scale and -Delta of the tile's rows
};

// MASK_DOC: qlist[0, nlist) holds the listed query tiles (DOC_MASK_FLAG: needs
// the element test), sQD the staged query documents, drow the batch row's ids;
// the caller has already staged iteration 0 (head 0, the diagonal tile qt0,
// which is always listed first) with dkdv_stage_first.
// MASK_KPM: qlist as above, drow the key-validity row, fv the first valid
// key's position: query rows before it (guarded) see every key, other rows
// need the key valid and not after them.
template <typename T, int D, bool DSROLE, int MODE, bool STORE, bool PART>
__device__ __forceinline__ void dkdv_role(
    DkdvStage<T, D>* st, u32x4* sP, const T* __restrict__ krot, const T* __restrict__ v,
    const T* __restrict__ qrot, const T* __restrict__ dout,
    const float* __restrict__ lse2, const float* __restrict__ delta,
    const float* __restrict__ cos, const float* __restrict__ sin, T* __restrict__ dk,
    T* __restrict__ dv, int S, int P, int Hq, int Hkv, int n_rep, int b, int g, int bh, int k0,
    int w, int lane, float scale_log2, float scale, int causal, const int32_t* __restrict__ drow,
    const uint16_t* qlist, int nlist, int32_t (*sQD)[BQ], int fv, u32x4* __restrict__ dsb,
    int nqtp, bool live, int part, int nsplit, float* __restrict__ pout) {
  constexpr bool DOC = MODE == MASK_DOC, KPM = MODE == MASK_KPM, LIST = DOC || KPM;
  // key padding keeps records only for a batch row whose first key is valid:
  // it has no guarded rows, so every dS tile lies in the causal record layout
  const bool keep = STORE && (!KPM || fv == 0);
  constexpr int KS = D / 16, DT = D / 32, HALF = D / 2;
  constexpr int KR = D / 8;
  // fragment reads run PF MFMAs ahead (2 in the masked modes, whose lists and
  // masks take the registers of a third)
  constexpr int PF = LIST ? 2 : 3;
  // the dS waves' phase 2 when they keep records: 2 ahead (its four dS
  // registers stay live to the end of the tile, for the deferred store)
  constexpr int PF2 = DSROLE && STORE ? 2 : PF;
  const int hh = lane >> 5, c32 = lane & 31;
  const int kw = w & 3;
  const int key = k0 + 32 * kw + c32;

  const int nqt = (S + BQ - 1) / BQ;
  const int qt0 = causal ? k0 / BQ : 0;
  const int per_head = LIST ? nlist : nqt - qt0;
  // (live false: no query tile, dK / dV stored as zeros; a later launch
  // writes this item's results)
  // PART: part `part` of `nsplit` takes the group's query heads
  // [h_base, h_base + n_rep / nsplit); otherwise all n_rep
  const int nh = PART ? n_rep / nsplit : n_rep, h_base = PART ? part * nh : 0;
  const int total = per_head > 0 && live ? per_head * nh : 0;
  // iteration -> query tile entry (tile | DOC_MASK_FLAG when listed), head-major
  auto entry = [&](int it) -> int {
    return LIST ? __builtin_amdgcn_readfirstlane((int)qlist[it % per_head]) : qt0 + it % per_head;
  };
  auto tile_of = [](int e) -> int { return LIST ? e & ~DOC_MASK_FLAG : e; };
  // DOC: this lane's key's document; KPM: 1 if this lane's key is valid
  const int kdoc = DOC ? drow[min(key, S - 1)] : KPM ? (key < S && drow[min(key, S - 1)] != 0) : 0;

  const uint32_t st_lds = lds_addr(st);
  auto stage_tile = [&](int hl, int qtile, int buf) {
    const int hq = g * n_rep + hl;
    const int64_t bhq = (int64_t)b * Hq + hq;
    const int q0 = qtile * BQ;
    DkdvStage<T, D>& S_ = st[buf];
    // (the masked modes recompute the per-lane offsets per tile: their lists
    // and masks leave no registers to keep them in)
    tile_to_lds<BQ, KR, 8, LIST>(qrot + (bhq * P + q0) * D, D, S_.q, w, lane);
    // dO in place ([B, S, Hq, D]): rows past S repeat row S - 1 (their lse is
    // +inf, so they contribute nothing)
    tile_to_lds<BQ, KR, 8, LIST>(dout + (((int64_t)b * S + q0) * Hq + hq) * D, Hq * D, S_.o, w,
                                 lane, S - q0);
    if (LIST || PART) {
      // the row statistics' LDS addresses from the stage array's base plus
      // constant offsets: with the pointer into the stage member, the masked
      // and split kernels fail to compile ("Operand has incorrect register
      // class": a constant generic-to-LDS address cast lowered with an
      // illegal null test)
      using Stage = DkdvStage<T, D>;
      const uint32_t sb = st_lds + (uint32_t)(buf * sizeof(Stage));
      if (w == 0) dma4(sb + offsetof(Stage, l), (uint32_t)lane * 4u, lse2 + bhq * P + q0);
      if (w == 1) dma4(sb + offsetof(Stage, dl), (uint32_t)lane * 4u, delta + bhq * P + q0);
    } else {
      if (w == 0) row_to_lds(lse2 + bhq * P + q0, S_.l, lane);
      if (w == 1) row_to_lds(delta + bhq * P + q0, S_.dl, lane);
    }
    if (DOC && w == 2) dma4(lds_addr(sQD[buf]), (uint32_t)min(q0 + lane, S - 1) * 4u, drow);
  };
  auto stage = [&](int it, int buf) {
    stage_tile(h_base + it / per_head, tile_of(entry(it)), buf);
  };
  // DOC: the first tile was staged by the caller before the list was built
  if (!DOC && total > 0) stage(0, 0);

  // this role's register-resident B operand: K (rotated, workspace rows up to P)
  // for P waves, V (read in place, [B, S, Hkv, D]; zero past S) for dS waves
  bf16x8 bf[KS];
  {
    // (masked modes: key and half laundered, so that the 64-bit row address
    // is formed here per item rather than hoisted out of the persistent loop
    // and kept in scratch)
    const int key_l = key;
    int hh_l = hh;
    if (LIST) asm volatile("" : "+v"(hh_l));
    const bool ok = !DSROLE || key_l < S;
    const T* src = DSROLE ? v + (((int64_t)b * S + (ok ? key_l : 0)) * Hkv + g) * D + 8 * hh_l
                             : krot + ((int64_t)bh * P + key_l) * D + 8 * hh_l;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      bf[ks] = as_bf16x8(ok ? *(const u32x4*)(src + 16 * ks) : u32x4{0u, 0u, 0u, 0u});
  }
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

  // A-operand tiles of the two products of this role
  auto first_tile = [](const DkdvStage<T, D>& S_) -> const T* { return DSROLE ? S_.o : S_.q; };
  auto second_tile = [](const DkdvStage<T, D>& S_) -> const T* { return DSROLE ? S_.q : S_.o; };
  u32x4* myP = sP + kw * 4 * 64 + lane;  // chunk c at myP[c * 64]
  const TrOffsets<D> tro = tr_offsets<D>(lane);

  // STORE (dS waves): each dS tile goes to its record after the tile's end
  // (non-temporal: the records are read once, by the dQ kernel).  The record's
  // index is scalar work done before the mid-tile barrier, where the dS waves
  // wait for P anyway, not between dS and the dK products.
  const int k32 = k0 / DSK + kw;  // this wavefront's 32-key record column
  const int nqtp2 = 2 * nqtp;
  const int64_t rec_bh = (int64_t)bh * nqtp * (causal ? nqtp + 1 : nqtp2);
  int rec_head = h_base, rec_tile = 0;  // head and tile count of iteration it (no division)

  lds_copy_wait();
  __syncthreads();
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) settle(bf[ks]);
  // the tile loop unrolled by two, so that each copy's LDS buffer is a
  // compile-time constant: fragment addresses are then loop-invariant per lane
  auto tile_body = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    if (it + 1 < total) stage(it + 1, buf ^ 1);
    const DkdvStage<T, D>& S_ = st[buf];
    const int e = entry(it);
    const int q0 = tile_of(e) * BQ;
    const int rel = key - q0;  // rows r of this tile see the key when r >= rel
    const bool diag = causal && q0 < k0 + BKV;
    const bool dmask = LIST && (e & DOC_MASK_FLAG);

    // this lane's 32 rows' -lse / scale (P waves) or -Delta (dS waves), the
    // start of the phase-1 accumulation (the first MFMA's C operand, so the
    // registers are free for the rest of the tile).  Element 4 gq + j of half
    // mt is row 32 mt + 8 gq + 4 hh + j, the row of the C-layout element
    // x[mt][4 gq + j].
    f32x16 rowv[2];
    {
      const float* src = DSROLE ? S_.dl : S_.l;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const f32x4 r4 = *(const f32x4*)(&src[32 * mt + 8 * gq + 4 * hh]);
#pragma unroll
          for (int j = 0; j < 4; ++j) rowv[mt][4 * gq + j] = r4[j];
        }
    }

    // phase 1: S - lse / scale (P waves) or dP - Delta (dS waves) for both
    // 32-row halves
    f32x16 x[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      x[mt] = rowv[mt];
      const T* tA = first_tile(S_);
      bf16x8 fa[KS];
#pragma unroll
      for (int ks = 0; ks < PF; ++ks) fa[ks] = lds_frag<KR>(tA, 32 * mt + c32, 2 * ks + hh);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        __builtin_amdgcn_sched_barrier(0);
        if (ks + PF < KS) fa[ks + PF] = lds_frag<KR>(tA, 32 * mt + c32, 2 * (ks + PF) + hh);
        x[mt] = mfma32<T>(fa[ks], bf[ks], x[mt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    u32x4 pk[4];
    if (!DSROLE) {
      // the causal test only on diagonal tiles (a uniform branch, not a
      // per-element select on every tile)
      auto make_p = [&](auto masked) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int r0 = 32 * mt + 8 * gq + 4 * hh;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float p = fast_exp2(x[mt][4 * gq + j] * scale_log2);
              if (decltype(masked)::value) p = (rel > r0 + j) ? 0.f : p;
              v[j] = p;
            }
            if (DOC && dmask) {
              const i32x4 qd = *(const i32x4*)&sQD[buf][r0];
#pragma unroll
              for (int j = 0; j < 4; ++j) v[j] = qd[j] != kdoc ? 0.f : v[j];
            }
            if (KPM && dmask) {
              // guarded rows keep every key; the others need it valid and not later
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const bool guarded = q0 + r0 + j < fv;
                v[j] = (!guarded && (rel > r0 + j || !kdoc)) ? 0.f : v[j];
              }
            }
            pk[2 * mt + (gq >> 1)][2 * (gq & 1)] = pack2<T>(v[0], v[1]);
            pk[2 * mt + (gq >> 1)][2 * (gq & 1) + 1] = pack2<T>(v[2], v[3]);
          }
      };
      if (!(KPM && dmask) && diag)
        make_p(std::true_type{});
      else
        make_p(std::false_type{});
#pragma unroll
      for (int c = 0; c < 4; ++c) myP[c * 64] = pk[c];
    }
    bf16x8 fpre[PF2];  // dS waves: first phase-2 fragments, read before the barrier
    // record of this tile (-1: above the causal diagonal, nothing to keep)
    int64_t rec = -1;
    if (STORE && DSROLE && keep) {
      const int qt = q0 / DSQ;
      if (!causal || k32 <= 2 * qt + 1)
        rec = ((rec_bh + (causal ? (int64_t)qt * (qt + 1) : (int64_t)qt * nqtp2) + k32) * n_rep +
               rec_head) * 256;
      asm volatile("" : "+s"(rec));
    }
    if (DSROLE) {
      // the first dK fragments while P is still on its way: only the product
      // with P is left between the barrier and the dK products
      asm volatile("" : "+v"(x[0]), "+v"(x[1]));
#pragma unroll
      for (int n = 0; n < PF2; ++n) fpre[n] = lds_frag_t<D>(second_tile(S_), tro, n / DT, n % DT);
    }
    __syncthreads();  // P of this tile is in LDS
    if (DSROLE) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          const u32x4 pp = myP[(2 * mt + cc) * 64];
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int gq = 2 * cc + half;
            float v[4];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              unpack2<T>(pp[2 * half + j], v[2 * j], v[2 * j + 1]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] *= x[mt][4 * gq + j];
            pk[2 * mt + cc][2 * half] = pack2<T>(v[0], v[1]);
            pk[2 * mt + cc][2 * half + 1] = pack2<T>(v[2], v[3]);
          }
        }
    }
    // phase 2: dV^T += dO^T P (P waves) or dK^T += Q^T dS (dS waves)
    {
      constexpr int NS = 4 * DT;
      const T* tA = second_tile(S_);
      bf16x8 fa[NS];
#pragma unroll
      for (int n = 0; n < PF2; ++n)
        fa[n] = DSROLE ? fpre[n] : lds_frag_t<D>(tA, tro, n / DT, n % DT);
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        __builtin_amdgcn_sched_barrier(0);
        if (n + PF2 < NS)
          fa[n + PF2] = lds_frag_t<D>(tA, tro, (n + PF2) / DT, (n + PF2) % DT);
        acc[n % DT] = mfma32<T>(fa[n], as_bf16x8(pk[n / DT]), acc[n % DT]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (STORE && ++rec_tile == per_head) {
      rec_tile = 0;
      ++rec_head;
    }
    lds_copy_wait();
    __syncthreads();
    // the dS record leaves after the end-of-tile wait: vmcnt counts stores
    // with the staging loads, so a store issued inside the tile holds every
    // wavefront at that wait until it is written; issued here it has the
    // next tile's duration to complete
    if (DSROLE && STORE && rec >= 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) __builtin_nontemporal_store(pk[c], dsb + rec + c * 64 + lane);
    }
  };
  for (int it = 0; it < total; it += 2) {
    tile_body(it, std::integral_constant<int, 0>{});
    if (it + 1 < total) tile_body(it + 1, std::integral_constant<int, 1>{});
  }

  if (key >= S) return;
  if (PART) {
    // a part of a split item: this role's float32 sums (dK or dV; the
    // reduction applies the scale, the RoPE backward and the rounding);
    // element 4 gi + e of acc[dt] is dim 32 dt + 8 gi + 4 hh + e
    float* dst = pout + ((int64_t)bh * S + key) * D + 4 * hh;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi)
        *(f32x4*)(dst + 32 * dt + 8 * gi) =
            f32x4{acc[dt][4 * gi], acc[dt][4 * gi + 1], acc[dt][4 * gi + 2], acc[dt][4 * gi + 3]};
    return;
  }
  const int key_e = key;
  int hoff = 4 * hh;
  if (LIST) asm volatile("" : "+v"(hoff));
  if (DSROLE) {
    T* dkr = dk + (((int64_t)b * S + key_e) * Hkv + g) * D + hoff;
    const float* cr = cos + (int64_t)key_e * HALF + hoff;
    const float* sr = sin + (int64_t)key_e * HALF + hoff;
#pragma unroll
    for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = 32 * dt + 8 * gi;
        float lo[4], hi[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rope_pair_bwd<T>(acc[dt][4 * gi + e] * scale, acc[dt + DT / 2][4 * gi + e] * scale,
                              cr[d + e], sr[d + e], lo[e], hi[e]);
        *(u32x2*)(dkr + d) = u32x2{pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3])};
        *(u32x2*)(dkr + d + HALF) = u32x2{pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3])};
      }
  } else {
    T* dvr = dv + (((int64_t)b * S + key_e) * Hkv + g) * D + hoff;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = 32 * dt + 8 * gi;
        *(u32x2*)(dvr + d) = u32x2{pack2<T>(acc[dt][4 * gi], acc[dt][4 * gi + 1]),
                                   pack2<T>(acc[dt][4 * gi + 2], acc[dt][4 * gi + 3])};
      }
  }
}

// Stage query tile q0 of query head bhq into buffer 0 (what dkdv_role's
// iteration 0 reads) with its document ids.
template <typename T, int D>
__device__ __forceinline__ void dkdv_stage_first(
    DkdvStage<T, D>* st, const T* __restrict__ qrot, const T* __restrict__ dout,
    const float* __restrict__ lse2, const float* __restrict__ delta,
    const int32_t* __restrict__ drow, int S, int P, int Hq, int b, int hq, int q0, int32_t* sqd,
    int w, int lane) {
  constexpr int KR = D / 8;
  const int64_t bhq = (int64_t)b * Hq + hq;
  tile_to_lds<BQ, KR, 8>(qrot + (bhq * P + q0) * D, D, st[0].q, w, lane);
  tile_to_lds<BQ, KR, 8>(dout + (((int64_t)b * S + q0) * Hq + hq) * D, Hq * D, st[0].o, w, lane,
                         S - q0);
  if (w == 0) row_to_lds(lse2 + bhq * P + q0, st[0].l, lane);
  if (w == 1) row_to_lds(delta + bhq * P + q0, st[0].dl, lane);
  if (w == 2) dma4(lds_addr(sqd), (uint32_t)min(q0 + lane, S - 1) * 4u, drow);
}

// kpm_flags (causal key padding; per batch row, 1 = every key valid): rows
// without padding run the unmasked kernel (SPLIT), the others the KPM one,
// which runs after it and skips the rows without padding; the unmasked launch
// walks no query tile for the padded rows' items (their dK / dV are written
// as zeros, then overwritten by the KPM launch).
template <typename T, int D, int MODE, bool STORE, bool SPLIT = false, bool PART = false>
__global__ __launch_bounds__(512, 1) void bwd_dkdv_kernel(
    const T* __restrict__ krot, const T* __restrict__ v, const T* __restrict__ qrot,
    const T* __restrict__ dout, const float* __restrict__ lse2, const float* __restrict__ delta,
    const float* __restrict__ cos, const float* __restrict__ sin, T* __restrict__ dk,
    T* __restrict__ dv, int S, int P, int Hq, int Hkv, int n_rep, int nkb, int nitems,
    float scale_log2,
    float scale, int causal, const int32_t* __restrict__ aux, const int2* __restrict__ ranges,
    u32x4* __restrict__ dsb, const int* __restrict__ order, const int* __restrict__ kpm_flags,
    int nsplit, float* __restrict__ dkp, float* __restrict__ dvp, int64_t part_stride) {
  constexpr bool DOC = MODE == MASK_DOC, KPM = MODE == MASK_KPM;
  __shared__ __attribute__((aligned(16))) DkdvStage<T, D> st[2];
  __shared__ __attribute__((aligned(16))) u32x4 sP[4 * 4 * 64];  // [key group][chunk][lane]
  __shared__ __attribute__((aligned(16))) int32_t sQD[2][BQ];   // DOC: query document ids
  __shared__ uint16_t sList[DOC_MAX_TILES];                      // listed query tiles
  __shared__ int sCount, sFirst;
  const int w = wave_id(), lane = threadIdx.x & 63;
  // persistent: one (key block, KV head) item per round; PART: an item is one
  // of nsplit parts of a key block, each with n_rep / nsplit of the group's
  // query heads (unmasked kernels only)
  const XcdItems xi = xcd_items(nitems);
  for (int rnd = 0;; ++rnd) {
    // PART (the small-grid variant): the shares dealt longest first over all
    // (KV head, part) groups of nkb key blocks
    int logical = xcd_item(xi, rnd);
    if (logical < 0) break;
    if (PART) logical = dealt_order(logical, nitems, nkb);
    // PART items are numbered (KV head, part, key block), key blocks fastest,
    // so an XCD's contiguous share holds whole longest-first sweeps of key
    // blocks (wavefront-uniform; readfirstlane keeps the staging bases scalar)
    int part = 0;
    if (PART) {
      const int kbl = logical % nkb, t = logical / nkb;
      part = __builtin_amdgcn_readfirstlane(t % nsplit);
      logical = __builtin_amdgcn_readfirstlane((t / nsplit) * nkb + kbl);
    }
    if (order != nullptr) {
      // items by descending work (the (batch row, key block) order, heads
      // adjacent), dealt round-robin over the XCDs
      const int rank = (logical - xi.lo) * 8 + (int)(blockIdx.x % 8);
      const int bk = order[rank / Hkv];
      logical = ((bk / nkb) * Hkv + rank % Hkv) * nkb + bk % nkb;
    }
    const int bh = logical / nkb;
    const int kb = logical % nkb;  // ascending: the longest causal key tiles first
    const int b = bh / Hkv, g = bh % Hkv;
    const int k0 = kb * BKV;
    const int32_t* drow = DOC || KPM ? aux + (int64_t)b * S : nullptr;
    const int2* rec = ranges + (int64_t)b * (P / BN);
    if (KPM && kpm_flags != nullptr && kpm_flags[b] != 0) continue;
    const bool live = !SPLIT || kpm_flags[b] != 0;
    int nlist = 0, fv = 0;
    if constexpr (KPM) {
      if (w == 0) {
        const int f = kpm_first_valid(rec, P / BN, lane);
        // valid keys in this block (its two 64-key tiles) against its keys below S
        const int t0 = k0 / BN;
        const int nval = rec[t0].x + (t0 + 1 < P / BN ? rec[t0 + 1].x : 0);
        const int nkeys = min(BKV, S - k0);
        const int qt0 = k0 / BQ;
        // query tiles holding guarded rows, then the causal ones if a key is valid
        const int n = kpm_tile_list(
            rec, 0, (S + BQ - 1) / BQ,
            [&](int t, int2) {
              return t * BQ < f ? 2 : (t >= qt0 && nval > 0) ? (nval < nkeys ? 2 : 1) : 0;
            },
            sList, lane);
        if (lane == 0) {
          sCount = n;
          sFirst = f;
        }
      }
      __syncthreads();
      nlist = __builtin_amdgcn_readfirstlane(sCount);
      fv = __builtin_amdgcn_readfirstlane(sFirst);
    }
    if constexpr (DOC) {
      const int qt0 = k0 / BQ;  // the diagonal query tile: always listed, first
      dkdv_stage_first<T, D>(st, qrot, dout, lse2, delta, drow, S, P, Hq, b, g * n_rep,
                          qt0 * BQ, sQD[0], w, lane);
      if (w == 0) {
        const int n = doc_tile_list(drow, k0, min(k0 + BKV, S), ranges + (int64_t)b * (P / BN),
                                    qt0, (S + BQ - 1) / BQ, sList, lane);
        if (lane == 0) sCount = n;
      }
      __syncthreads();
      nlist = __builtin_amdgcn_readfirstlane(sCount);
    }
    if (w >= 4)
      dkdv_role<T, D, true, MODE, STORE, PART>(st, sP, krot, v, qrot, dout, lse2, delta, cos, sin, dk,
                                      dv, S, P, Hq, Hkv, n_rep, b, g, bh, k0, w, lane,
                                      scale_log2, scale, causal, drow, sList, nlist, sQD, fv,
                                      dsb, P / DSQ, live, part, nsplit,
                                      PART ? dkp + part * part_stride : nullptr);
    else
      dkdv_role<T, D, false, MODE, STORE, PART>(st, sP, krot, v, qrot, dout, lse2, delta, cos, sin, dk,
                                       dv, S, P, Hq, Hkv, n_rep, b, g, bh, k0, w, lane,
                                       scale_log2, scale, causal, drow, sList, nlist, sQD, fv,
                                       dsb, P / DSQ, live, part, nsplit,
                                       PART ? dvp + part * part_stride : nullptr);
    __syncthreads();  // LDS of this item is free for the next
  }
}

// dK and dV of split dK/dV items: the nsplit parts' float32 sums added in
// part order, then what the unsplit kernel does at its store (dV rounded to T;
// dK scaled, rotated back by the dtype-cast tables, rounded).  Row r = bh * S
// + key; per row HALF / 4 threads take four dK dims and their RoPE partners,
// D / 8 threads eight dV dims.
template <typename T, int D>
__global__ __launch_bounds__(256) void dkdv_reduce_kernel(
    const float* __restrict__ dkp, const float* __restrict__ dvp, int nsplit,
    int64_t part_stride, const float* __restrict__ cos, const float* __restrict__ sin,
    T* __restrict__ dk, T* __restrict__ dv, int S, int Hkv, float scale, int nrows) {
  constexpr int HALF = D / 2, TK = HALF / 4, TPR = TK + D / 8;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int row = t / TPR, j = t % TPR;
  if (row >= nrows) return;
  const int bh = row / S, key = row % S, b = bh / Hkv, g = bh % Hkv;
  const int64_t out = (((int64_t)b * S + key) * Hkv + g) * D;
  const int64_t in = (int64_t)row * D;
  if (j < TK) {
    const int d0 = 4 * j;
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    for (int p = 0; p < nsplit; ++p) {
      lo += *(const f32x4*)(dkp + p * part_stride + in + d0);
      hi += *(const f32x4*)(dkp + p * part_stride + in + d0 + HALF);
    }
    float r1[4], r2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      rope_pair_bwd<T>(lo[e] * scale, hi[e] * scale, cos[(int64_t)key * HALF + d0 + e],
                       sin[(int64_t)key * HALF + d0 + e], r1[e], r2[e]);
    *(u32x2*)(dk + out + d0) = u32x2{pack2<T>(r1[0], r1[1]), pack2<T>(r1[2], r1[3])};
    *(u32x2*)(dk + out + d0 + HALF) = u32x2{pack2<T>(r2[0], r2[1]), pack2<T>(r2[2], r2[3])};
  } else {
    const int d0 = 8 * (j - TK);
    f32x4 a = {0.f, 0.f, 0.f, 0.f}, c = a;
    for (int p = 0; p < nsplit; ++p) {
      a += *(const f32x4*)(dvp + p * part_stride + in + d0);
      c += *(const f32x4*)(dvp + p * part_stride + in + d0 + 4);
    }
    *(u32x4*)(dv + out + d0) = u32x4{pack2<T>(a[0], a[1]), pack2<T>(a[2], a[3]),
                                     pack2<T>(c[0], c[1]), pack2<T>(c[2], c[3])};
  }
}

// dQ workgroup: 8 wavefronts x 32 rows = 256 (query head, position) rows of one
// KV group, all sharing each staged K / V / K^T tile (two wavefronts per SIMD).
// DOC walks the listed key tiles last to first, like the forward.
constexpr int DQ_ROWS = 256;

template <typename T, int D, int MODE>
__global__ __launch_bounds__(512, 1) void bwd_dq_kernel(
    const T* __restrict__ qrot, const T* __restrict__ dout, const float* __restrict__ lse2,
    const float* __restrict__ delta, const T* __restrict__ krot, const T* __restrict__ v,
    const float* __restrict__ cos, const float* __restrict__ sin, T* __restrict__ dq, int S,
    int P, int Hq, int Hkv, int n_rep, int bm_pos, int nqb, int nitems, float scale_log2,
    float scale, int causal, const int32_t* __restrict__ aux, const int2* __restrict__ ranges,
    int kpm_skip_clean) {
  constexpr bool DOC = MODE == MASK_DOC, KPM = MODE == MASK_KPM, LIST = DOC || KPM;
  constexpr int KS = D / 16, DT = D / 32, HALF = D / 2;
  constexpr int KR = D / 8;
  struct Stage {
    T k[BN * D], v[BN * D];
  };
  __shared__ __attribute__((aligned(16))) Stage st[2];
  __shared__ __attribute__((aligned(16))) int32_t sKD[2][BN];  // LIST: per-key aux values
  __shared__ uint16_t sList[DOC_MAX_TILES];                     // LIST: listed key tiles
  __shared__ int sCount, sFirst;

  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63, hh = lane >> 5, c32 = lane & 31;
  // persistent: one block of rows per round
  const XcdItems xi = xcd_items(nitems);
  for (int rnd = 0;; ++rnd) {
    const int logical = xcd_item(xi, rnd);
    if (logical < 0) break;
    // kpm_skip_clean: the batch rows whose key 0 is valid have their dQ from
    // the dS records (bwd_dq_ds); this launch serves the others
    if (KPM && kpm_skip_clean &&
        __builtin_amdgcn_readfirstlane(ranges[(int64_t)(logical / nqb / Hkv) * (P / BN)].y) == 0)
      continue;
    // per-lane values laundered per item: hoisted out of the persistent loop,
    // the row split and the per-lane 64-bit bases derived from them would be
    // kept in scratch across the item
    int r_l = w * 32 + c32, lane_l = lane;
    asm volatile("" : "+v"(r_l), "+v"(lane_l));
    const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, S, r_l);
    const int bh = ri.b * Hkv + ri.g;
    const int64_t bhq = (int64_t)ri.b * Hq + ri.hq;

    const int kend = causal ? min(S, ri.p0 + bm_pos) : S;
    int ntiles = (kend + BN - 1) / BN;
    const int32_t* drow = LIST ? aux + (int64_t)ri.b * S : nullptr;
    const int2* rec = ranges + (int64_t)ri.b * (P / BN);
    const T* kbase = krot + (int64_t)bh * P * D;
    // V read in place ([B, S, Hkv, D]); rows past S repeat row S - 1 (their K
    // rows are zero, so they add nothing to dQ)
    const T* vbase = v + ((int64_t)ri.b * S * Hkv + ri.g) * D;
    auto stage = [&](int t, int buf) {
      tile_to_lds<BN, KR, 8, true>(kbase + (int64_t)t * BN * D, D, st[buf].k, w, lane);
      tile_to_lds<BN, KR, 8, true>(vbase + (int64_t)t * BN * Hkv * D, Hkv * D, st[buf].v, w, lane,
                                   S - t * BN);
      if (LIST && w == 0) dma4(lds_addr(sKD[buf]), (uint32_t)min(t * BN + lane, S - 1) * 4u, drow);
    };
    int di = 0;        // DOC: this row's document
    bool grd = false;  // KPM: this row is guarded (before the first valid key)
    if constexpr (DOC) {
      // walked backwards, as in the forward: the always-listed last tile loads
      // while the list is built
      if (ntiles > 0) stage(ntiles - 1, 0);
      di = drow[min(ri.pos, S - 1)];
      if (w == 0) {
        const int n = doc_tile_list(drow, ri.p0, min(ri.p0 + bm_pos, S), rec, 0, ntiles, sList,
                                    lane_l);
        if (lane == 0) sCount = n;
      }
      __syncthreads();
      ntiles = __builtin_amdgcn_readfirstlane(sCount);
    } else if constexpr (KPM) {
      const int nall = (S + BN - 1) / BN;
      if (w == 0) {
        const int f = kpm_first_valid(rec, P / BN, lane);
        const bool guard_block = ri.p0 < f;  // a guarded row needs every key tile
        const int n = kpm_tile_list(rec, 0, guard_block ? nall : ntiles,
                                    [&](int, int2 r) { return guard_block ? 2 : r.x == 0 ? 0 : r.x < BN ? 2 : 1; },
                                    sList, lane_l);
        if (lane == 0) {
          sCount = n;
          sFirst = f;
        }
      }
      __syncthreads();
      ntiles = __builtin_amdgcn_readfirstlane(sCount);
      grd = ri.pos < sFirst;
    } else {
      if (ntiles > 0) stage(0, 0);
    }
    auto entry = [&](int it) -> int {
      return DOC ? __builtin_amdgcn_readfirstlane((int)sList[ntiles - 1 - it])
                 : KPM ? __builtin_amdgcn_readfirstlane((int)sList[it]) : it;
    };
    auto tile_of = [](int e) -> int { return LIST ? e & ~DOC_MASK_FLAG : e; };
    if (KPM && ntiles > 0) stage(tile_of(entry(0)), 0);

    bf16x8 qf[KS], df[KS];
    float l2 = INFINITY, ndl = 0.f;  // ndl: -Delta of this lane's row
    if (ri.q_valid) {
      const int hoff = 8 * (lane_l >> 5);
      const T* qr = qrot + (bhq * P + ri.pos) * D + hoff;
      const T* dr = dout + (((int64_t)ri.b * S + ri.pos) * Hq + ri.hq) * D + hoff;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = as_bf16x8(*(const u32x4*)(qr + 16 * ks));
        df[ks] = as_bf16x8(*(const u32x4*)(dr + 16 * ks));
      }
      l2 = -lse2[bhq * P + ri.pos] * scale_log2;  // lse log2(e) from -lse / scale
      ndl = delta[bhq * P + ri.pos];
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
        df[ks] = qf[ks];
      }
    }

    f32x16 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;
    const TrOffsets<D> tro = tr_offsets<D>(lane);

    lds_copy_wait();
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      settle(qf[ks]);
      settle(df[ks]);
    }
    settle(l2);
    settle(ndl);
    for (int it = 0; it < ntiles; ++it) {
      const int buf = it & 1;
      const int e = entry(it);
      const int t = tile_of(e);
      if (it + 1 < ntiles) stage(tile_of(entry(it + 1)), buf ^ 1);
      const Stage& S_ = st[buf];
      const int k0 = t * BN;
      const bool dmask = LIST && (e & DOC_MASK_FLAG);
      const bool need_mask = (causal && k0 + BN - 1 > ri.p0) || (k0 + BN > S) || dmask;
      // last visible key of this lane's row, relative to k0 (a guarded row: any below S)
      const int lim = (causal && !grd ? min(ri.pos, S - 1) : S - 1) - k0;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x16 s, dp;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[i] = 0.f;
          dp[i] = 0.f;
        }
        {
          // fragment reads run PF steps ahead of the MFMAs that consume them
          constexpr int PF = 2;
          bf16x8 fk[KS], fv[KS];
#pragma unroll
          for (int ks = 0; ks < PF; ++ks) {
            fk[ks] = lds_frag<KR>(S_.k, 32 * mt + c32, 2 * ks + hh);
            fv[ks] = lds_frag<KR>(S_.v, 32 * mt + c32, 2 * ks + hh);
          }
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            __builtin_amdgcn_sched_barrier(0);
            if (ks + PF < KS) {
              fk[ks + PF] = lds_frag<KR>(S_.k, 32 * mt + c32, 2 * (ks + PF) + hh);
              fv[ks + PF] = lds_frag<KR>(S_.v, 32 * mt + c32, 2 * (ks + PF) + hh);
            }
            s = mfma32<T>(fk[ks], qf[ks], s);
            dp = mfma32<T>(fv[ks], df[ks], dp);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        u32x4 dsk[2];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          float dsv[2];
          // DOC: documents of this pair's two keys (adjacent: i even)
          int kd[2] = {0, 0};
          if (dmask) {
            const int local0 = 32 * mt + 8 * (i >> 2) + 4 * hh + (i & 3);
            kd[0] = sKD[buf][local0];
            kd[1] = sKD[buf][local0 + 1];
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            float p = fast_exp2(__builtin_fmaf(s[i + j], scale_log2, -l2));
            if (need_mask) {
              const int local = 32 * mt + 8 * ((i + j) >> 2) + 4 * hh + ((i + j) & 3);
              p = local > lim ? 0.f : p;
              if (DOC && dmask) p = kd[j] != di ? 0.f : p;
              if (KPM && dmask && !grd) p = kd[j] == 0 ? 0.f : p;
            }
            dsv[j] = p * (dp[i + j] + ndl);
          }
          dsk[i >> 3][(i & 7) >> 1] = pack2<T>(dsv[0], dsv[1]);
        }
        {
          constexpr int NS = 2 * DT, PF = 1;
          bf16x8 fa[NS];
#pragma unroll
          for (int n = 0; n < PF; ++n)
            fa[n] = lds_frag_t<D>(S_.k, tro, 2 * mt + n / DT, n % DT);
#pragma unroll
          for (int n = 0; n < NS; ++n) {
            __builtin_amdgcn_sched_barrier(0);
            if (n + PF < NS)
              fa[n + PF] = lds_frag_t<D>(S_.k, tro, 2 * mt + (n + PF) / DT, (n + PF) % DT);
            acc[n % DT] = mfma32<T>(fa[n], as_bf16x8(dsk[n / DT]), acc[n % DT]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      lds_copy_wait();
      __syncthreads();
    }

    if (ri.q_valid) {
      T* dqr = dq + (((int64_t)ri.b * S + ri.pos) * Hq + ri.hq) * D;
      const int hoff = 4 * (lane_l >> 5);
      const float* cr = cos + (int64_t)ri.pos * HALF + hoff;
      const float* sr = sin + (int64_t)ri.pos * HALF + hoff;
#pragma unroll
      for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = 32 * dt + 8 * gi;
          float lo[4], hi[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            rope_pair_bwd<T>(acc[dt][4 * gi + e] * scale, acc[dt + DT / 2][4 * gi + e] * scale,
                                cr[d + e], sr[d + e], lo[e], hi[e]);
          *(u32x2*)(dqr + d + hoff) = u32x2{pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3])};
          *(u32x2*)(dqr + d + hoff + HALF) = u32x2{pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3])};
        }
    }
    __syncthreads();  // LDS of this item is free for the next
  }
}

// dma16 with the nontemporal (streaming) cache policy, for data read once
__device__ __forceinline__ void dma16_nt(uint32_t lds, uint32_t voff, const void* base) {
  asm volatile(KF_VMEM_ASM_NOPS "global_load_lds_dwordx4 %0, %1 nt"
               : : "v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// dQ from the dS records: workgroup = HB query heads of one KV group x DSQ
// positions, one wavefront per head (its 64 rows as two 32-row blocks, so each
// K^T fragment feeds two products).  Per DSK-key step it stages the rotated K
// rows [DSK][D] and the HB records into LDS (a ring of NBUF, loads issued
// NBUF - 1 steps ahead: 4 for short sequences with 4 heads per workgroup,
// where one workgroup per CU with three steps in flight does best, otherwise 3,
// two workgroups per CU with two steps each) and accumulates dQ^T += K^T dS^T: K^T comes from the K
// rows by ds_read_b64_tr_b16 (lds_frag_t), dS^T from the records by the same
// instruction, which turns a record's one-key-per-lane layout into one row per
// lane.  The kernel moves the dS bytes once and does one product per element;
// it is bound by HBM.  With packed documents (DOC) the steps walk only the key
// tiles listed for the query tile, two record columns per 64-key tile; with key
// padding (KPM) the causal tiles holding a valid key, in batch rows whose key 0
// is valid (the others are left to the recompute kernel).
template <typename T, int D, int HB, int MODE, int NBUF>
__global__ __launch_bounds__(64 * HB) void bwd_dq_ds_kernel(
    const u32x4* __restrict__ dsb, const T* __restrict__ krot, const float* __restrict__ cos,
    const float* __restrict__ sin, T* __restrict__ dq, int S, int P, int Hq, int Hkv,
    int n_rep, int nqt, int causal, float scale, const int32_t* __restrict__ doc,
    const int2* __restrict__ ranges) {
  constexpr bool DOC = MODE == MASK_DOC, KPM = MODE == MASK_KPM, LIST = DOC || KPM;
  constexpr int NW = HB, KR = D / 8, DT = D / 32, HALF = D / 2;
  static_assert(NBUF == 3 || NBUF == 4, "ring depth");
  constexpr int KI = DSK * KR / 64;  // 1 KB load instructions per K step
  static_assert(KI % NW == 0, "K rows must split evenly over the wavefronts");
  // load instructions per wavefront and step: its share of K, its record's 4 KB
  constexpr int NLOAD = KI / NW + 4;
  struct Stage {
    T k[DSK * D];
    u32x4 ds[HB * 256];
  };
  __shared__ __attribute__((aligned(16))) Stage st[NBUF];
  const int w = wave_id(), lane = threadIdx.x & 63, hh = lane >> 5, c32 = lane & 31;
  // item (KV head, head group, query tile), a KV head's tiles numbered
  // longest-causal-row first, dealt to the XCDs by xcd_logical_id
  const int ngrp = n_rep / HB;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqt);
  const int qt = nqt - 1 - logical % nqt;
  const int hg = (logical / nqt) % ngrp, bh = logical / nqt / ngrp;
  const int b = bh / Hkv, g = bh % Hkv;
  const int nqtp = P / DSQ;
  int nk = causal ? min(2 * qt + 2, (S + DSK - 1) / DSK) : (S + DSK - 1) / DSK;
  // DOC: the 64-key tiles whose document range meets this tile's rows (the
  // dK/dV pass listed this query tile for their key blocks, so their records
  // exist); each listed tile is two steps.  Causal: tiles 0 .. qt.
  // KPM: the tiles 0 .. qt with a valid key (the dK/dV pass listed this query
  // tile for every key block holding one), when the batch row's key 0 is valid
  __shared__ uint16_t sList[LIST ? DS_DOC_MAX_TILES : 1];
  __shared__ int sCount;
  if constexpr (KPM) {
    const int2* rec = ranges + (int64_t)b * (P / BN);
    if (__builtin_amdgcn_readfirstlane(rec[0].y) != 0) return;  // guarded rows: dq's
    if (w == 0) {
      const int n = kpm_tile_list(rec, 0, qt + 1, [](int, int2 r) { return r.x > 0 ? 1 : 0; },
                                  sList, lane);
      if (lane == 0) sCount = n;
    }
    __syncthreads();
    nk = 2 * __builtin_amdgcn_readfirstlane(sCount);
  }
  if constexpr (DOC) {
    if (w == 0) {
      const int n = doc_tile_list(doc + (int64_t)b * S, qt * DSQ, min(qt * DSQ + DSQ, S),
                                  ranges + (int64_t)b * (P / BN), 0, qt + 1, sList, lane);
      if (lane == 0) sCount = n;
    }
    __syncthreads();
    nk = 2 * __builtin_amdgcn_readfirstlane(sCount);
  }
  // record column (32 keys) of step t
  auto col = [&](int t) -> int {
    return LIST ? 2 * (__builtin_amdgcn_readfirstlane((int)sList[t >> 1]) & ~DOC_MASK_FLAG) + (t & 1)
                : t;
  };
  const u32x4* rec0 = dsb + (ds_pair(bh, qt, 0, nqtp, causal) * n_rep + hg * HB) * 256;
  const T* kbase = krot + (int64_t)bh * P * D;
  auto stage = [&](int t_, int buf) {
    const int t = col(t_);
#pragma unroll
    for (int jj = 0; jj < KI / NW; ++jj) {
      const int j = w * (KI / NW) + jj;
      const int L = j * 64 + lane, row = L / KR, pc = L % KR;
      const uint32_t off =
          ((uint32_t)(t * DSK + row) * D + (uint32_t)(pc ^ swz<KR>(row)) * 8u) * 2u;
      dma16(lds_addr(st[buf].k + j * 512), off, kbase);
    }
    // this wavefront's record (read once: streaming loads), 4 x 1 KB of 64
    // 16-byte B-operand pieces; lane i of LDS copy j takes piece
    // (i ^ 8 (j & 1)) ^ 4 (i >> 5): the 4 (i >> 5) term puts the two 16-lane
    // groups of a transposed read's pass that share a copy in different halves
    // of a 256-byte bank window, the 8 (j & 1) term (128 bytes) does the same
    // for the two groups that read copies j and j + 1
    const u32x4* src = rec0 + ((int64_t)t * n_rep + w) * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dma16_nt(lds_addr(st[buf].ds + w * 256 + j * 64),
               (uint32_t)((j * 64 + ((lane ^ (8 * (j & 1))) ^ ((lane >> 5) << 2))) * 16), src);
  };

  // transposed-read address of this lane inside its record (row block mh adds
  // 2048 bytes, key chunk c 256, the second read of a chunk 128, which the odd
  // copies hold 128 bytes lower): address-lane 4e + k of group G fetches rows
  // 16(G&1) + 4k .. +3 of key 4(G>>1) + e
  uint32_t ds_off;
  {
    const int G = lane >> 4, a = lane & 15, e = a >> 2, k = a & 3;
    const int piece = 32 * (k & 1) + 4 * ((G >> 1) ^ (k & 1)) + e;
    ds_off = (uint32_t)(w * 4096 + (G & 1) * (1024 + 128) + piece * 16 + 8 * (k >> 1));
  }
  const TrOffsets<D> tro = tr_offsets<D>(lane);
  f32x16 acc[2][DT];
#pragma unroll
  for (int mh = 0; mh < 2; ++mh)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mh][dt][i] = 0.f;

#pragma unroll
  for (int t = 0; t < NBUF - 1; ++t)
    if (t < nk) stage(t, t);
  for (int t = 0; t < nk; ++t) {
    // step t's loads are in; those of up to NBUF - 2 later steps may still fly
    const int ahead = min(NBUF - 2, nk - 1 - t);
    if (ahead >= 2)
      vm_wait<2 * NLOAD>();
    else if (ahead == 1)
      vm_wait<NLOAD>();
    else
      vm_wait<0>();
    __syncthreads();  // every wavefront's share landed; step t - 1's buffer is free
    if (t + NBUF - 1 < nk) stage(t + NBUF - 1, (t + NBUF - 1) % NBUF);
    const Stage& S_ = st[t % NBUF];
    const char* dsl = (const char*)S_.ds + ds_off;
    const char* dsh = (const char*)S_.ds + (ds_off ^ 128u);
#pragma unroll
    for (int c = 0; c < DSK / 16; ++c) {
      bf16x8 bds[2];
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        const int o = 2048 * mh + 256 * c;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(dsl + o));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(dsh + o));
        bds[mh] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5,
                                                                     6, 7));
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 ak = lds_frag_t<D>(S_.k, tro, c, dt);
#pragma unroll
        for (int mh = 0; mh < 2; ++mh)
          acc[mh][dt] =
              mfma32<T>(ak, bds[mh], acc[mh][dt]);
      }
    }
  }

  const int hq = g * n_rep + hg * HB + w;
  // dQ leaves through LDS (the ring is free once every wavefront is past its
  // last products): each wavefront writes its 64 rows into its own 64 x D
  // slice, 16-byte chunks XOR-swizzled by row, then stores whole chunks, KR
  // consecutive lanes per row, instead of 8 bytes of each of 32 rows.
  static_assert(HB * 64 * D * 2 <= NBUF * (int)sizeof(Stage), "dQ slices exceed the ring");
  __syncthreads();
  T* slice = (T*)st + w * 64 * D;
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    const int r = 32 * mh + c32;
    const int pos = min(qt * DSQ + r, S - 1);  // rows past S are formed, not stored
    const float* cr = cos + (int64_t)pos * HALF;
    const float* sr = sin + (int64_t)pos * HALF;
#pragma unroll
    for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = 32 * dt + 8 * gi + 4 * hh;
        float lo[4], hi[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rope_pair_bwd<T>(acc[mh][dt][4 * gi + e] * scale,
                              acc[mh][dt + DT / 2][4 * gi + e] * scale, cr[d + e], sr[d + e],
                              lo[e], hi[e]);
        const int cl = 4 * dt + gi, chh = KR / 2 + 4 * dt + gi;  // chunks of d and d + HALF
        *(u32x2*)(slice + (r * KR + (cl ^ (r & (KR - 1)))) * 8 + 4 * hh) =
            u32x2{pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3])};
        *(u32x2*)(slice + (r * KR + (chh ^ (r & (KR - 1)))) * 8 + 4 * hh) =
            u32x2{pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3])};
      }
  }
  __syncthreads();
#pragma unroll
  for (int i2 = 0; i2 < KR; ++i2) {
    const int L = 64 * i2 + lane, r = L / KR, ch = L % KR;
    const int pos = qt * DSQ + r;
    const u32x4 v = *(const u32x4*)(slice + (r * KR + (ch ^ (r & (KR - 1)))) * 8);
    if (pos < S) *(u32x4*)(dq + (((int64_t)b * S + pos) * Hq + hq) * D + 8 * ch) = v;
  }
}

// dQ from the dS records, two query tiles per workgroup (unmasked causal
// launches, head_dim 128, 4 query heads per workgroup): 8 wavefronts, one per
// (tile, head); the tiles are adjacent (2p, 2p + 1), so they share the staged
// K rows of every step but the later tile's last two.  Per step the stage
// holds the K rows (8 KB, one load per wavefront) and the 8 records (4 KB
// each); a ring of three stages, two steps in flight.  Against one tile per
// workgroup: half the K-row traffic and half the workgroups (their start-up
// and epilogue), and two wavefronts per SIMD.  A wavefront whose tile has no
// record at a step (the earlier tile at the later tile's last two steps)
// loads its last record again (the load counts stay equal across wavefronts)
// and skips the products.
template <typename T, int D, int NBUF>
__global__ __launch_bounds__(512) void bwd_dq_ds2_kernel(
    const u32x4* __restrict__ dsb, const T* __restrict__ krot, const float* __restrict__ cos,
    const float* __restrict__ sin, T* __restrict__ dq, int S, int P, int Hq, int Hkv,
    int n_rep, int nqt, float scale) {
  constexpr int HB = 4, NW = 8, KR = D / 8, DT = D / 32, HALF = D / 2;
  constexpr int KI = DSK * KR / 64;  // 1 KB load instructions per K step
  static_assert(KI % NW == 0, "K rows must split evenly over the wavefronts");
  constexpr int NLOAD = KI / NW + 4;
  struct Stage {
    T k[DSK * D];
    u32x4 ds[NW * 256];
  };
  constexpr int RING_B = NBUF * (int)sizeof(Stage), OUT_B = NW * 64 * D * 2;
  __shared__ __attribute__((aligned(16))) char smem[RING_B > OUT_B ? RING_B : OUT_B];
  Stage* st = (Stage*)smem;
  const int w = wave_id(), lane = threadIdx.x & 63, hh = lane >> 5, c32 = lane & 31;
  const int hw = w % HB, tw = w / HB;
  const int npair = (nqt + 1) / 2, ngrp = n_rep / HB;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, npair);
  const int pp = npair - 1 - logical % npair;  // longest causal rows first
  const int hg = (logical / npair) % ngrp, bh = logical / npair / ngrp;
  const int b = bh / Hkv, g = bh % Hkv;
  const int nqtp = P / DSQ;
  const int qt = 2 * pp + tw;
  const bool live = qt < nqt;  // (the second tile of an odd last pair does not exist)
  const int qt_last = min(2 * pp + 1, nqt - 1);
  const int nkeys = (S + DSK - 1) / DSK;
  const int nk = min(2 * qt_last + 2, nkeys);            // steps of the workgroup
  const int nk_w = live ? min(2 * qt + 2, nkeys) : 0;   // steps with a record of this wave
  const u32x4* rec0 = dsb + (ds_pair(bh, live ? qt : qt_last, 0, nqtp, 1) * n_rep + hg * HB + hw) * 256;
  const T* kbase = krot + (int64_t)bh * P * D;
  auto stage = [&](int t, int buf) {
    const int L = w * 64 + lane, row = L / KR, pc = L % KR;  // KI / NW == 1
    const uint32_t off = ((uint32_t)(t * DSK + row) * D + (uint32_t)(pc ^ swz<KR>(row)) * 8u) * 2u;
    dma16(lds_addr(st[buf].k + w * 512), off, kbase);
    // this wavefront's record of column t (its last one again past its steps);
    // the piece permutation of bwd_dq_ds_kernel
    const int tr = min(t, max(nk_w, 1) - 1);
    const u32x4* src = rec0 + (int64_t)tr * n_rep * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dma16_nt(lds_addr(st[buf].ds + w * 256 + j * 64),
               (uint32_t)((j * 64 + ((lane ^ (8 * (j & 1))) ^ ((lane >> 5) << 2))) * 16), src);
  };
  uint32_t ds_off;
  {
    const int G = lane >> 4, a = lane & 15, e = a >> 2, k = a & 3;
    const int piece = 32 * (k & 1) + 4 * ((G >> 1) ^ (k & 1)) + e;
    ds_off = (uint32_t)(w * 4096 + (G & 1) * (1024 + 128) + piece * 16 + 8 * (k >> 1));
  }
  const TrOffsets<D> tro = tr_offsets<D>(lane);
  f32x16 acc[2][DT];
#pragma unroll
  for (int mh = 0; mh < 2; ++mh)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mh][dt][i] = 0.f;

#pragma unroll
  for (int t = 0; t < NBUF - 1; ++t)
    if (t < nk) stage(t, t);
  for (int t = 0; t < nk; ++t) {
    const int ahead = min(NBUF - 2, nk - 1 - t);
    if (ahead >= 2)
      vm_wait<2 * NLOAD>();
    else if (ahead == 1)
      vm_wait<NLOAD>();
    else
      vm_wait<0>();
    __syncthreads();
    if (t + NBUF - 1 < nk) stage(t + NBUF - 1, (t + NBUF - 1) % NBUF);
    if (t < nk_w) {
      const Stage& S_ = st[t % NBUF];
      const char* dsl = (const char*)S_.ds + ds_off;
      const char* dsh = (const char*)S_.ds + (ds_off ^ 128u);
#pragma unroll
      for (int c = 0; c < DSK / 16; ++c) {
        bf16x8 bds[2];
#pragma unroll
        for (int mh = 0; mh < 2; ++mh) {
          const int o = 2048 * mh + 256 * c;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(dsl + o));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(dsh + o));
          bds[mh] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5,
                                                                       6, 7));
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 ak = lds_frag_t<D>(S_.k, tro, c, dt);
#pragma unroll
          for (int mh = 0; mh < 2; ++mh)
            acc[mh][dt] =
                mfma32<T>(ak, bds[mh], acc[mh][dt]);
        }
      }
    }
  }

  // dQ through LDS, every wavefront's 64 rows in its own slice of the ring
  const int hq = g * n_rep + hg * HB + hw;
  __syncthreads();
  T* slice = (T*)smem + w * 64 * D;
#pragma unroll
  for (int mh = 0; mh < 2; ++mh) {
    const int r = 32 * mh + c32;
    const int pos = min(qt * DSQ + r, S - 1);  // rows past S are formed, not stored
    const float* cr = cos + (int64_t)pos * HALF;
    const float* sr = sin + (int64_t)pos * HALF;
#pragma unroll
    for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = 32 * dt + 8 * gi + 4 * hh;
        float lo[4], hi[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rope_pair_bwd<T>(acc[mh][dt][4 * gi + e] * scale,
                              acc[mh][dt + DT / 2][4 * gi + e] * scale, cr[d + e], sr[d + e],
                              lo[e], hi[e]);
        const int cl = 4 * dt + gi, chh = KR / 2 + 4 * dt + gi;
        *(u32x2*)(slice + (r * KR + (cl ^ (r & (KR - 1)))) * 8 + 4 * hh) =
            u32x2{pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3])};
        *(u32x2*)(slice + (r * KR + (chh ^ (r & (KR - 1)))) * 8 + 4 * hh) =
            u32x2{pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3])};
      }
  }
  __syncthreads();
  if (!live) return;
#pragma unroll
  for (int i2 = 0; i2 < KR; ++i2) {
    const int L = 64 * i2 + lane, r = L / KR, ch = L % KR;
    const int pos = qt * DSQ + r;
    const u32x4 v = *(const u32x4*)(slice + (r * KR + (ch ^ (r & (KR - 1)))) * 8);
    if (pos < S) *(u32x4*)(dq + (((int64_t)b * S + pos) * Hq + hq) * D + 8 * ch) = v;
  }
}

// MASK_DOC: how many tiles each block of a workgroup's rows lists, i.e. the
// work of the item it takes; one wavefront per block.  Key side (rows = keys):
// the query tiles from the block's diagonal tile to the end; query side: the
// key tiles from 0 to the last one the block's rows can see (causal).  ranges
// is [B][rstride] per 64-position tile; counts[b * nblk + i] for block i.
__global__ __launch_bounds__(256) void doc_block_tiles_kernel(
    const int32_t* __restrict__ doc, const int2* __restrict__ ranges, int S, int rstride,
    int rows, int nblk, int nitems, int key_side, int* __restrict__ counts) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + w;
  if (i >= nitems) return;
  const int b = i / nblk, p0 = (i % nblk) * rows, p1 = min(p0 + rows, S);
  const int t0 = key_side ? p0 / BN : 0;
  const int t1 = key_side ? (S + BN - 1) / BN : (p1 + BN - 1) / BN;
  const int n = doc_tile_list(doc + (int64_t)b * S, p0, p1, ranges + (int64_t)b * rstride, t0, t1,
                              nullptr, lane);
  if (lane == 0) counts[i] = n;
}

// The blocks by descending count (a counting sort in one workgroup): the
// workgroup of rank r takes the r-th, so the hardware's in-order dispatch
// deals the longest items first and each XCD (every 8th rank) an equal share.
// Ties land in any order; no result depends on which workgroup computes an item.
__global__ __launch_bounds__(1024) void order_by_count_kernel(const int* __restrict__ counts,
                                                              int n, int* __restrict__ order) {
  __shared__ int hist[DOC_MAX_TILES + 1];
  const int t = threadIdx.x;
  for (int c = t; c <= DOC_MAX_TILES; c += 1024) hist[c] = 0;
  __syncthreads();
  for (int i = t; i < n; i += 1024) atomicAdd(&hist[min(counts[i], DOC_MAX_TILES)], 1);
  __syncthreads();
  if (t < 64) {
    // start of each count's run in descending order: lane t sums PER bins from
    // the top, then an exclusive prefix of the lane sums
    constexpr int PER = (DOC_MAX_TILES + 1 + 63) / 64;
    int local[PER], sum = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = DOC_MAX_TILES - (PER * t + j);
      local[j] = c >= 0 ? hist[c] : 0;
      sum += local[j];
    }
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (t >= o) incl += v;
    }
    int run = incl - sum;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = DOC_MAX_TILES - (PER * t + j);
      if (c >= 0) hist[c] = run;
      run += local[j];
    }
  }
  __syncthreads();
  for (int i = t; i < n; i += 1024) order[atomicAdd(&hist[min(counts[i], DOC_MAX_TILES)], 1)] = i;
}

}  // namespace

int launch_doc_order(const int32_t* doc, const int2* ranges, int S, int rstride, int rows, int B,
                     int nblk, int key_side, int* counts, int* order, hipStream_t stream) {
  const int nitems = B * nblk;
  KF_LAUNCH("doc_block_tiles", doc_block_tiles_kernel, dim3((nitems + 3) / 4), dim3(256), 0,
            stream, doc, ranges, S, rstride, rows, nblk, nitems, key_side, counts);
  KF_LAUNCH("order_by_count", order_by_count_kernel, dim3(1), dim3(1024), 0, stream, counts,
            nitems, order);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

namespace {

struct Ws {
  uint16_t *krot, *qrot;  // 16-bit elements of the call's dtype
  float *lse2, *delta;  // -lse / scale and -Delta (q_prep_bwd)
  float* dkvp;  // split dK/dV items: nsplit dK parts, then nsplit dV parts, [B*Hkv][S][D] each
  int2* ranges;  // [B][P/64] document-id range per tile (packed documents only)
  int *counts, *order;  // [B][P/128] each: dK/dV item work and order (packed documents)
  u32x4* dsb;    // dS records (when kept)
};

// Parts each unmasked dK/dV item is split into.  The persistent grid has one
// workgroup per CU and its zigzag shares pair long items with short ones, so
// it needs at least two items per workgroup; a launch with fewer (few batch
// rows and KV heads: a tensor-parallel rank's share, long single sequences)
// gives each part of an item an equal share of the KV group's query heads
// (the smallest divisor of n_rep up to 8 that reaches two items per
// workgroup, else the largest), and dkdv_reduce_kernel adds the parts'
// float32 sums.  Measured without the split on the reference's TP = 4
// shares, the dK/dV kernel took 2.9x (70B) and 5.4x (29B) its C3 time per
// causal pair.  The masked kernels are not persistent and are not split (key
// padding's unpadded batch rows run the unmasked kernel, split the same way).
int dkdv_splits(int B, int S, int Hq, int Hkv) {
  const int n_rep = Hq / Hkv;
  const int64_t items = (int64_t)(pad_len(S) / BKV) * B * Hkv;
  const int64_t want = 2 * (int64_t)(device_cu_count() / 8 * 8);
  if (items >= want) return 1;
  int n = 1;
  for (int d = 2; d <= 8 && d <= n_rep; ++d) {
    if (n_rep % d) continue;
    n = d;
    if (items * d >= want) break;
  }
  return n;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Whether the unmasked dK/dV launch takes the small-grid variant (PART):
// split items, or KV heads that do not fill the 8 XCDs in whole groups (its
// shares are then dealt by lane_order).  It writes float32 parts that
// dkdv_reduce_kernel adds (one part when unsplit).
bool dkdv_small_grid(int B, int S, int Hq, int Hkv) {
  return dkdv_splits(B, S, Hq, Hkv) > 1 || (B * Hkv) % 8 != 0;
}

// the small-grid variant's float32 dK and dV parts (none otherwise)
size_t split_bytes(int B, int S, int Hq, int Hkv, int D) {
  if (!dkdv_small_grid(B, S, Hq, Hkv)) return 0;
  return 2 * (size_t)dkdv_splits(B, S, Hq, Hkv) * B * Hkv * S * D * sizeof(float);
}

// krot and qrot (unless the caller's rot holds them), lse2, delta, tile
// records, item counts and order, then (256-byte aligned) the split dK/dV parts
size_t base_bytes(int B, int S, int Hq, int Hkv, int D, bool rot) {
  const size_t P = (size_t)pad_len(S);
  const size_t head = (rot ? 0 : ((size_t)B * Hkv + (size_t)B * Hq) * P * D * sizeof(uint16_t)) +
                      2 * (size_t)B * Hq * P * sizeof(float) +
                      (size_t)B * (P / BN) * sizeof(int2) + 2 * (size_t)B * (P / BKV) * sizeof(int);
  const size_t parts = split_bytes(B, S, Hq, Hkv, D);
  return parts ? align256(head) + parts : head;
}

// Largest dS record store the backward uses; past it dQ recomputes S and dP.
constexpr size_t DS_STORE_MAX = (size_t)32 << 30;

// bytes of the dS records of this launch, or 0 when they are not kept
size_t ds_bytes(const BwdArgs& a) {
  // key padding: the causal layout only (its batch rows without guarded rows)
  if ((a.kvalid && !a.causal) || ((a.doc || a.kvalid) && pad_len(a.S) / DSQ > DS_DOC_MAX_TILES))
    return 0;
  const size_t nqtp = (size_t)pad_len(a.S) / DSQ;
  const size_t pairs = a.causal ? nqtp * (nqtp + 1) : 2 * nqtp * nqtp;
  const size_t bytes = (size_t)a.B * a.Hq * pairs * 4096;
  return bytes <= DS_STORE_MAX ? bytes : 0;
}

Ws carve(void* base, int B, int S, int Hq, int Hkv, int D, const void* rot) {
  const size_t P = (size_t)pad_len(S);
  const size_t kv = (size_t)B * Hkv * P * D, qq = (size_t)B * Hq * P * D;
  Ws w;
  uint16_t* p = rot ? (uint16_t*)rot : (uint16_t*)base;
  w.krot = p; p += kv;
  w.qrot = p; p += qq;
  float* f = rot ? (float*)base : (float*)p;
  w.lse2 = f; f += (size_t)B * Hq * P;
  w.delta = f; f += (size_t)B * Hq * P;
  w.ranges = (int2*)f;
  w.counts = (int*)(w.ranges + (size_t)B * (P / BN));
  w.order = w.counts + (size_t)B * (P / BKV);
  w.dkvp = (float*)((char*)base + align256((size_t)((char*)(w.order + (size_t)B * (P / BKV)) -
                                                    (char*)base)));
  w.dsb = (u32x4*)((char*)base + align256(base_bytes(B, S, Hq, Hkv, D, rot != nullptr)));
  return w;
}

template <typename T, int D, int HB>
int launch_dq_ds(const BwdArgs& a, const Ws& w) {
  const int P = pad_len(a.S), n_rep = a.Hq / a.Hkv, nqt = (a.S + DSQ - 1) / DSQ;
  // ring depth by sequence length (measured with 4 heads per workgroup: 4
  // buffers 485 against 517 us at S = 4096, 3115 against 2967 at S = 16384)
  const bool deep = HB == 4 && a.S <= 8192;
  // two query tiles per workgroup for the long sequences (measured: C5 2910 us
  // against 2959; at S = 4096 one tile with four stages does better, 468
  // against 491)
  if constexpr (D == 128 && HB == 4)
  if (!a.doc && !a.kvalid && a.causal && !deep) {
    const int npair = (nqt + 1) / 2;
    KF_LAUNCH("bwd_dq_ds", (bwd_dq_ds2_kernel<T, D, 3>), dim3(a.B * a.Hkv * (n_rep / HB) * npair),
              dim3(512), 0, a.stream, w.dsb, (const T*)w.krot, a.cos, a.sin, (T*)a.dq, a.S, P,
              a.Hq, a.Hkv, n_rep, nqt, a.scale);
    KF_CHECK_LAUNCH();
    return KF_OK;
  }
  KF_LAUNCH("bwd_dq_ds",
            (a.doc      ? (deep ? bwd_dq_ds_kernel<T, D, HB, MASK_DOC, 4>
                                : bwd_dq_ds_kernel<T, D, HB, MASK_DOC, 3>)
             : a.kvalid ? (deep ? bwd_dq_ds_kernel<T, D, HB, MASK_KPM, 4>
                                : bwd_dq_ds_kernel<T, D, HB, MASK_KPM, 3>)
                        : (deep ? bwd_dq_ds_kernel<T, D, HB, MASK_NONE, 4>
                                : bwd_dq_ds_kernel<T, D, HB, MASK_NONE, 3>)),
            dim3(a.B * a.Hkv * (n_rep / HB) * nqt), dim3(64 * HB), 0, a.stream, w.dsb,
            (const T*)w.krot, a.cos, a.sin, (T*)a.dq, a.S, P, a.Hq, a.Hkv, n_rep, nqt, a.causal,
            a.scale, a.doc, w.ranges);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <typename T, int D>
int launch_bwd(const BwdArgs& a, void* workspace, bool keep_ds) {
  const int P = pad_len(a.S);
  const Ws w = carve(workspace, a.B, a.S, a.Hq, a.Hkv, D, a.rot);
  const int n_rep = a.Hq / a.Hkv;
  const float scale_log2 = a.scale * kLog2e;
  FwdArgs fa{};
  fa.k = a.k; fa.v = a.v; fa.cos = a.cos; fa.sin = a.sin;
  fa.B = a.B; fa.Sq = a.S; fa.Sk = a.S; fa.Hq = a.Hq; fa.Hkv = a.Hkv; fa.D = D;
  fa.ksb = fa.vsb = (int64_t)a.S * a.Hkv * D;
  fa.kss = fa.vss = (int64_t)a.Hkv * D;
  fa.ksh = fa.vsh = D;
  fa.k_rotated = 0; fa.dtype = dtype_code<T>(); fa.stream = a.stream;
  fa.doc = a.doc; fa.kvalid = a.kvalid; fa.causal = a.causal;
  // with a.rot the rotated K and Q are the forward's: only the tile records of
  // an explicit mask are left to prepare
  if (!a.rot || a.doc || a.kvalid) {
    const int rc = launch_kv_prep(fa, a.rot ? nullptr : w.krot, P, nullptr, P, w.ranges, KV_V_NONE);
    if (rc) return rc;
  }
  KF_LAUNCH("q_prep_bwd", (q_prep_bwd_kernel<T, D>), dim3(P / BN, a.B * a.Hq), dim3(256), 0,
            a.stream, a.rot ? nullptr : (const T*)a.q, (const T*)a.out, (const T*)a.dout, a.lse,
            a.cos, a.sin, (T*)w.qrot, w.lse2, w.delta, a.S, P, a.Hq, 1.f / a.scale);
  KF_CHECK_LAUNCH();
  const int nkb = P / BKV;
  // packed documents: the dK/dV items by their listed query tiles, most first
  const int* order = nullptr;
  if (a.doc) {
    const int rc = launch_doc_order(a.doc, w.ranges, a.S, P / BN, BKV, a.B, nkb, 1, w.counts,
                                    w.order, a.stream);
    if (rc) return rc;
    order = w.order;
  }
  // persistent grids: one workgroup per CU (a multiple of 8, one share per XCD).
  // With an explicit mask the items' lengths no longer fall in launch order, so
  // the zigzag shares would not balance: one workgroup per item there.
  const int grid_cap = a.doc || a.kvalid ? INT_MAX : device_cu_count() / 8 * 8;
  const int mode = a.doc ? MASK_DOC : a.kvalid ? MASK_KPM : MASK_NONE;
  const int32_t* aux = a.doc ? a.doc : a.kvalid;
  // causal key padding: the batch rows whose keys are all valid go to the
  // unmasked (persistent) kernel first, the rest to the KPM one
  const int* kpm_flags = mode == MASK_KPM && a.causal ? w.counts : nullptr;
  // Small grids (dkdv_small_grid) take the unmasked kernel's PART variant,
  // whose float32 parts dkdv_reduce adds; key padding's rows without padding
  // take the same variant as an unmasked launch, so an all-True mask gives the
  // unmasked result bit for bit
  const int64_t part_stride = (int64_t)a.B * a.Hkv * a.S * D;
  const bool small = dkdv_small_grid(a.B, a.S, a.Hq, a.Hkv);
  auto reduce_parts = [&](int nsplit, float* dkp, float* dvp) {
    constexpr int TPR = D / 8 + D / 8;  // threads per row of dkdv_reduce_kernel
    const int64_t nrows = (int64_t)a.B * a.Hkv * a.S;
    KF_LAUNCH("dkdv_reduce", (dkdv_reduce_kernel<T, D>),
              dim3((unsigned)((nrows * TPR + 255) / 256)), dim3(256), 0, a.stream, dkp, dvp,
              nsplit, part_stride, a.cos, a.sin, (T*)a.dk, (T*)a.dv, a.S, a.Hkv, a.scale,
              (int)nrows);
  };
  if (kpm_flags) {
    const int rc = launch_kpm_row_flags(w.ranges, P / BN, a.S, a.B, w.counts, a.stream);
    if (rc) return rc;
    const int ns = dkdv_splits(a.B, a.S, a.Hq, a.Hkv);
    float* dkp = small ? w.dkvp : nullptr;
    float* dvp = small ? w.dkvp + ns * part_stride : nullptr;
    const int ni = nkb * a.B * a.Hkv * ns;
    KF_LAUNCH("bwd_dkdv",
              (small ? (keep_ds ? bwd_dkdv_kernel<T, D, MASK_NONE, true, true, true>
                                 : bwd_dkdv_kernel<T, D, MASK_NONE, false, true, true>)
                      : (keep_ds ? bwd_dkdv_kernel<T, D, MASK_NONE, true, true>
                                 : bwd_dkdv_kernel<T, D, MASK_NONE, false, true>)),
              dim3(std::min(ni, device_cu_count() / 8 * 8)), dim3(512), 0, a.stream,
              (const T*)w.krot, (const T*)a.v, (const T*)w.qrot, (const T*)a.dout, w.lse2, w.delta,
              a.cos, a.sin, (T*)a.dk, (T*)a.dv, a.S, P, a.Hq, a.Hkv, n_rep, nkb, ni, scale_log2,
              a.scale, a.causal, nullptr, w.ranges, w.dsb, nullptr, kpm_flags, ns, dkp, dvp,
              part_stride);
    if (small) reduce_parts(ns, dkp, dvp);
  }
  const int nsplit = mode == MASK_NONE ? dkdv_splits(a.B, a.S, a.Hq, a.Hkv) : 1;
  const bool part = mode == MASK_NONE && small;
  float* dkp = part ? w.dkvp : nullptr;
  float* dvp = part ? w.dkvp + nsplit * part_stride : nullptr;
  const int nitems = nkb * a.B * a.Hkv * nsplit;
  KF_LAUNCH("bwd_dkdv",
            (mode == MASK_DOC   ? (keep_ds ? bwd_dkdv_kernel<T, D, MASK_DOC, true>
                                           : bwd_dkdv_kernel<T, D, MASK_DOC, false>)
             : mode == MASK_KPM ? (keep_ds ? bwd_dkdv_kernel<T, D, MASK_KPM, true>
                                           : bwd_dkdv_kernel<T, D, MASK_KPM, false>)
             : part             ? (keep_ds ? bwd_dkdv_kernel<T, D, MASK_NONE, true, false, true>
                                           : bwd_dkdv_kernel<T, D, MASK_NONE, false, false, true>)
             : keep_ds          ? bwd_dkdv_kernel<T, D, MASK_NONE, true>
                                : bwd_dkdv_kernel<T, D, MASK_NONE, false>),
            dim3(std::min(nitems, grid_cap)), dim3(512), 0, a.stream, (const T*)w.krot,
            (const T*)a.v, (const T*)w.qrot, (const T*)a.dout, w.lse2, w.delta, a.cos, a.sin,
            (T*)a.dk, (T*)a.dv, a.S, P, a.Hq, a.Hkv, n_rep, nkb, nitems, scale_log2, a.scale,
            a.causal, aux, w.ranges, w.dsb, order, kpm_flags, nsplit, dkp, dvp, part_stride);
  if (part) reduce_parts(nsplit, dkp, dvp);
  KF_CHECK_LAUNCH();
  if (keep_ds) {
    const int rc = n_rep % 4 == 0   ? launch_dq_ds<T, D, 4>(a, w)
                   : n_rep % 2 == 0 ? launch_dq_ds<T, D, 2>(a, w)
                                    : launch_dq_ds<T, D, 1>(a, w);
    // key padding: the batch rows with guarded rows still recompute their dQ
    // (the records launch skipped them; this one skips the rest)
    if (rc || mode != MASK_KPM) return rc;
  }
  const int bm_pos = DQ_ROWS / n_rep;
  const int nqb = (a.S + bm_pos - 1) / bm_pos;
  KF_LAUNCH("bwd_dq",
            (mode == MASK_DOC   ? bwd_dq_kernel<T, D, MASK_DOC>
             : mode == MASK_KPM ? bwd_dq_kernel<T, D, MASK_KPM>
                                : bwd_dq_kernel<T, D, MASK_NONE>),
            dim3(std::min(nqb * a.B * a.Hkv, grid_cap)), dim3(512), 0, a.stream, (const T*)w.qrot,
            (const T*)a.dout, w.lse2, w.delta, (const T*)w.krot, (const T*)a.v, a.cos, a.sin,
            (T*)a.dq, a.S, P,
            a.Hq, a.Hkv, n_rep, bm_pos, nqb, nqb * a.B * a.Hkv, scale_log2, a.scale, a.causal,
            aux, w.ranges, (int)keep_ds);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

}  // namespace

bool bwd_mfma_supported(const BwdArgs& a) {
  if (a.doc && a.kvalid) return false;  // one explicit mask kind at a time
  if ((a.doc || a.kvalid) && pad_len(a.S) / BN > DOC_MAX_TILES) return false;
  if ((a.dtype != BF16 && a.dtype != F16) || (a.D != 64 && a.D != 128)) return false;
  const int n_rep = a.Hq / a.Hkv;
  if (n_rep < 1 || n_rep > ROWS) return false;  // also bounds DQ_ROWS / n_rep >= 2
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  return al16(a.q) && al16(a.k) && al16(a.v) && al16(a.out) && al16(a.dout) && al16(a.dq) &&
         al16(a.dk) && al16(a.dv) && al16(a.cos) && al16(a.sin);
}

size_t bwd_mfma_workspace(int B, int S, int Hq, int Hkv, int D, bool rot) {
  return base_bytes(B, S, Hq, Hkv, D, rot);
}

size_t bwd_mfma_workspace_ds(const BwdArgs& a) {
  const size_t base = base_bytes(a.B, a.S, a.Hq, a.Hkv, a.D, a.rot != nullptr), ds = ds_bytes(a);
  return ds ? align256(base) + ds : base;
}

int bwd_mfma(const BwdArgs& a, void* workspace, size_t workspace_bytes) {
  KF_CHECK_ARG((int64_t)pad_len(a.S) / BN * (int64_t)a.B * a.Hq < (1LL << 31), "grid too large");
  const bool keep_ds = ds_bytes(a) != 0 && workspace_bytes >= bwd_mfma_workspace_ds(a);
  if (a.dtype == F16)
    return a.D == 128 ? launch_bwd<f16, 128>(a, workspace, keep_ds)
                      : launch_bwd<f16, 64>(a, workspace, keep_ds);
  return a.D == 128 ? launch_bwd<bf16, 128>(a, workspace, keep_ds)
                    : launch_bwd<bf16, 64>(a, workspace, keep_ds);
}

}  // namespace kf
