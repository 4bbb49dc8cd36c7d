// HIP kernels for gfx950 (CDNA4, wave64): hybrid fp16 SpMM and SDDMM.
//
// Three SpMM kernels, all writing every output element exactly once (no atomics, no zero-fill):
//   k_spmm_tasks    residual CSR.  A "lane group" of LPG lanes owns one task: a run of whole rows
//                   (the entries streamed flat, rows flushed as their end is crossed) or one piece
//                   of a long row.  Each lane holds VEC consecutive features (8, 4, 2 or 1:
//                   16-, 8-, 4- or 2-byte loads, by K and alignment), so one B row of K fp16 is
//                   fetched by K/VEC lanes; U nonzeros are in flight per lane; narrow groups are
//                   held to 2 or 4 waves per SIMD by dynamic LDS.  fp32 accumulation.  Replaces the reference residual kernels
//                   (TR-source/SpMM/mGCNkernel.cu:976-1171, spmm_utils/compute.h:27-240), which
//                   accumulate in fp16 and only handle K = 128.
//   k_spmm_fixup    sums the pieces of split rows in a fixed order (deterministic).
//   k_spmm_mfma_win one workgroup owns a 16-row window: dense 16x16 fp16 tiles (TC blocks and
//                   well-filled 2:4 group tiles) go through v_mfma_f32_16x16x16_f16 with the 16
//                   gathered B rows staged in LDS; the window's residual rows are summed in
//                   registers, added to the MFMA share read back from LDS, and each output row is
//                   stored once.  Replaces the reference TC and packed mma.sp kernels
//                   (mGCNkernel_online.cu:54-241, 812-933) and the add kernel (:1314-1324).
// SDDMM (no reference counterpart):
//   k_sddmm_tasks   residual entries: one lane group per task, per-entry dot products reduced
//                   across the group; 16-, 8-, 4- or 2-byte loads of X and Y by K and alignment.
//   k_sddmm_mfma32  one wave per dense 16x16 tile: D = X[16 window rows] . Y[16 tile columns]^T
//                   accumulated over K with gfx950's v_mfma_f32_16x16x32_f16 (both operands
//                   contiguous in K, 16-byte loads straight from global), sampled at the tile's
//                   stored entries; k_sddmm_mfma is the same with v_mfma_f32_16x16x16_f16 for K
//                   that is not a multiple of 8.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "half.hpp"
#include "kernels.hpp"

// This file is compiled once per part (see the Makefile): TRS_KERNEL_PART = 8, 4, 2, 1 builds the
// SpMM / SDDMM launchers and kernels of that load width, 0 (the default) the plan-lowering kernels
// and the dispatch between the widths, so the kernel templates build in parallel.
#ifndef TRS_KERNEL_PART
#define TRS_KERNEL_PART 0
#endif

namespace trs {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half16_t __attribute__((ext_vector_type(16)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// ------------------------------------------------------------------------------------------------
// SpMM / SDDMM kernels and their launchers (the width parts only).
#if TRS_KERNEL_PART > 0

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <int VEC>
struct BFrag;
template <>
struct BFrag<8> {
  half8_t v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const half8_t*>(p); }
  // non-temporal: the line is not kept in the caches for later readers
  __device__ __forceinline__ void load_nt(const uint16_t* p) {
    v = __builtin_nontemporal_load(reinterpret_cast<const half8_t*>(p));
  }
  __device__ __forceinline__ void zero() { v = half8_t{0, 0, 0, 0, 0, 0, 0, 0}; }
  __device__ __forceinline__ void fma(float (&acc)[8], float a) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(a, (float)v[i], acc[i]);
  }
  // v_dot2_f32_f16: two fp16 products (exact in fp32) added to an fp32 accumulator per instruction
  __device__ __forceinline__ float dot(const BFrag& o) const {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s = __builtin_amdgcn_fdot2(half2_t{v[2 * i], v[2 * i + 1]}, half2_t{o.v[2 * i], o.v[2 * i + 1]}, s, false);
    return s;
  }
};
template <>
struct BFrag<4> {
  half4_t v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const half4_t*>(p); }
  __device__ __forceinline__ void zero() { v = half4_t{0, 0, 0, 0}; }
  __device__ __forceinline__ void fma(float (&acc)[4], float a) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(a, (float)v[i], acc[i]);
  }
  __device__ __forceinline__ float dot(const BFrag& o) const {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      s = __builtin_amdgcn_fdot2(half2_t{v[2 * i], v[2 * i + 1]}, half2_t{o.v[2 * i], o.v[2 * i + 1]}, s, false);
    return s;
  }
};
template <>
struct BFrag<2> {
  half2_t v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const half2_t*>(p); }
  __device__ __forceinline__ void zero() { v = half2_t{0, 0}; }
  __device__ __forceinline__ void fma(float (&acc)[2], float a) const {
    acc[0] = __builtin_fmaf(a, (float)v[0], acc[0]);
    acc[1] = __builtin_fmaf(a, (float)v[1], acc[1]);
  }
  __device__ __forceinline__ float dot(const BFrag& o) const { return __builtin_amdgcn_fdot2(v, o.v, 0.f, false); }
};
template <>
struct BFrag<1> {
  _Float16 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = __builtin_bit_cast(_Float16, *p); }
  __device__ __forceinline__ void zero() { v = (_Float16)0; }
  __device__ __forceinline__ void fma(float (&acc)[1], float a) const { acc[0] = __builtin_fmaf(a, (float)v, acc[0]); }
  __device__ __forceinline__ float dot(const BFrag& o) const { return (float)v * (float)o.v; }
};

// NT: non-temporal (streaming) store, so written output does not evict gathered B rows from L2.
template <int VEC, bool NT = false>
__device__ __forceinline__ void store_vec(float* dst, const float (&acc)[VEC]) {
  if constexpr (VEC == 8) {
    const float4_t lo{acc[0], acc[1], acc[2], acc[3]}, hi{acc[4], acc[5], acc[6], acc[7]};
    if constexpr (NT) {
      __builtin_nontemporal_store(lo, reinterpret_cast<float4_t*>(dst));
      __builtin_nontemporal_store(hi, reinterpret_cast<float4_t*>(dst) + 1);
    } else {
      reinterpret_cast<float4_t*>(dst)[0] = lo;
      reinterpret_cast<float4_t*>(dst)[1] = hi;
    }
  } else if constexpr (VEC == 4) {
    const float4_t v{acc[0], acc[1], acc[2], acc[3]};
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(dst));
    else reinterpret_cast<float4_t*>(dst)[0] = v;
  } else if constexpr (VEC == 2) {
    const float2_t v{acc[0], acc[1]};
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<float2_t*>(dst));
    else reinterpret_cast<float2_t*>(dst)[0] = v;
  } else {
    if constexpr (NT) __builtin_nontemporal_store(acc[0], dst);
    else dst[0] = acc[0];
  }
}

// Element offset of row `row` (validated non-negative) in an operand with leading dimension ld
// (the host guarantees ld < 2^31): one 32 x 32 -> 64-bit multiply per gather.
__device__ __forceinline__ uint64_t row_offset(int32_t row, int64_t ld) {
  return (uint64_t)(uint32_t)row * (uint64_t)(uint32_t)ld;
}

// Fragment address of entry column c: row c of B at Bf (leading dimension ld) or, with HOT and
// c < 0, staged hot row ~c at Hf (leading dimension hld).  Selects, no branch: the gathers of a
// batch still issue back to back.
template <bool HOT>
__device__ __forceinline__ const uint16_t* gather_addr(const uint16_t* Bf, int64_t ld, const uint16_t* Hf,
                                                       int32_t hld, int32_t c) {
  if constexpr (HOT) {
    const bool h = c < 0;
    return (h ? Hf : Bf) + row_offset(h ? ~c : c, h ? (int64_t)hld : ld);
  } else {
    return Bf + row_offset(c, ld);
  }
}

template <bool NT, class T>
__device__ __forceinline__ T load_stream(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Workgroups are dispatched round-robin over the 8 XCDs (physical id i runs on XCD i % 8), and
// each XCD has its own L2.  Remap so that every XCD executes runs of `run` consecutive logical
// workgroups: neighbouring rows (which share B rows on mesh-like graphs) then share one L2, while
// runs still interleave across XCDs so heavy work spread along the order stays balanced.
// Bijective on [0, n): the first (n / (8 run)) * 8 run ids are permuted, the tail is unchanged.
__device__ __forceinline__ int xcd_remap(int i, int n, int run) {
  constexpr int kXcds = 8;
  if (run <= 1) return i;
  const int span = kXcds * run;
  const int full = (n / span) * span;
  if (i >= full) return i;
  const int x = i % kXcds, j = i / kXcds;
  return (j / run) * span + x * run + (j % run);
}

// Residual task of lane group `grp` of wave `wave` (GPW lane groups per wave, 4 waves per
// workgroup).  With per-XCD queues, workgroup i runs on XCD i mod kXcds and takes its tasks, in
// order, from that XCD's queue; otherwise the tasks form one list spread by xcd_remap.
// block / nblocks: the workgroup's index among the nblocks that serve this task list (the launch's
// own index and size, or the part of a fused launch, whose XCD is still block mod kXcds).
__device__ __forceinline__ int residual_task(const DevicePlan& P, int wave, int grp, int gpw, bool& valid,
                                             int block, int nblocks) {
  if (P.xcd_queues) {
    const int x = block % kXcds, k = block / kXcds;
    const int id = P.xq[x] + (k * 4 + wave) * gpw + grp;
    valid = id < P.xq[x + 1];
    return id;
  }
  const int id = (xcd_remap(block, nblocks, P.xcd_run) * 4 + wave) * gpw + grp;
  valid = id < P.ntasks;
  return id;
}

// Workgroups of 4 waves x gpw lane groups that cover the plan's residual tasks.
inline int residual_grid(const DevicePlan& P, int gpw) {
  const int gpb = 4 * gpw;
  if (!P.xcd_queues) return (P.ntasks + gpb - 1) / gpb;
  int most = 0;
  for (int x = 0; x < kXcds; ++x) most = std::max(most, (P.xq[x + 1] - P.xq[x] + gpb - 1) / gpb);
  return most * kXcds;
}

// Row pointers rowptr[row_begin .. row_end] of a multi-row task into the lane group's LDS slice:
// all loads are issued before the first store (indices clamped to the task's last pointer), so
// the preload costs one memory round trip instead of one per pointer each lane handles.
template <int LPG>
__device__ __forceinline__ void preload_rowptr(const int32_t* __restrict__ rowptr, int row_begin, int nrows, int li,
                                               int* rp) {
  constexpr int PER_LANE = (kTaskRows + 1 + LPG - 1) / LPG;
  int v[PER_LANE];
#pragma unroll
  for (int k = 0; k < PER_LANE; ++k) {
    const int j = li + k * LPG;
    v[k] = rowptr[row_begin + (j <= nrows ? j : nrows)];
  }
#pragma unroll
  for (int k = 0; k < PER_LANE; ++k)
    if (li + k * LPG <= nrows) rp[li + k * LPG] = v[k];
}

template <int VEC>
__device__ __forceinline__ void zero_acc(float (&acc)[VEC]) {
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
}

// Loads of one batch of U entries [p, p + U) of a stream ending at `end` (> p): column ids, fp16
// values and the gathered B fragments.  Every load is unconditional -- indices past the end are
// clamped to the last entry and lanes past K read features [0, VEC) -- so the batch issues as one
// run of loads with no branch between them (a load under a branch makes the compiler wait for
// all earlier loads first, leaving one gather in flight per wave).  Callers ignore the padded
// slots and lanes.
//
// With PF (pipelined) the stream runs one batch deep: the column ids and values of batch b + 1 are
// loaded right after batch b's gathers are issued, so they arrive while batch b is consumed and a
// batch costs one memory round trip (its gathers) instead of two.  Whether that pays depends on
// the shape (see the launchers): it costs registers and raises the number of requests in flight.
//
// G = 2 or 4: the stream is shared by an aligned group of G lanes (one quad or half-quad), which
// load the batch cooperatively -- lane j of the group loads entries p + j, p + j + G, ... -- and
// exchange them with DPP quad broadcasts.  Every load instruction of a wave then carries G times
// fewer column/value requests (a wave with 4-lane groups serves 16 tasks, whose streams sit in 16
// different cache lines).
template <int G>
__device__ __forceinline__ int group_bcast(int v, int k) {   // lane k's v, to every lane of the group
  static_assert(G == 2 || G == 4, "quad broadcasts");
  if constexpr (G == 4) {
    switch (k) {   // quad_perm [k, k, k, k]
      case 0: return __builtin_amdgcn_mov_dpp(v, 0x00, 0xf, 0xf, false);
      case 1: return __builtin_amdgcn_mov_dpp(v, 0x55, 0xf, 0xf, false);
      case 2: return __builtin_amdgcn_mov_dpp(v, 0xaa, 0xf, 0xf, false);
      default: return __builtin_amdgcn_mov_dpp(v, 0xff, 0xf, 0xf, false);
    }
  } else {
    switch (k) {   // quad_perm [k, k, 2 + k, 2 + k]
      case 0: return __builtin_amdgcn_mov_dpp(v, 0xa0, 0xf, 0xf, false);
      default: return __builtin_amdgcn_mov_dpp(v, 0xf5, 0xf, 0xf, false);
    }
  }
}

template <int VEC, int U, bool NT, int G = 0>
struct Batch {
  int32_t cc[U];
  uint16_t vh[U];
  BFrag<VEC> bb[U];
  // column ids and values of entries [p, p + U) of a stream [.., end), end > 0; slots at or past
  // `end` repeat entry end - 1
  __device__ __forceinline__ void load_a(const int32_t* __restrict__ col, const uint16_t* __restrict__ val, int p,
                                         int end) {
    if constexpr ((G == 2 || G == 4) && U % G == 0) {
      constexpr int R = U / G;
      const int j = (int)(threadIdx.x & (G - 1));
      int c[R], v[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int q = p + r * G + j < end ? p + r * G + j : end - 1;
        c[r] = load_stream<NT>(col + q);
        v[r] = load_stream<NT>(val + q);
      }
#pragma unroll
      for (int i = 0; i < U; ++i) {
        cc[i] = group_bcast<G>(c[i / G], i % G);
        vh[i] = (uint16_t)group_bcast<G>(v[i / G], i % G);
      }
    } else {
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int q = p + i < end ? p + i : end - 1;
        cc[i] = load_stream<NT>(col + q);
        vh[i] = load_stream<NT>(val + q);
      }
    }
  }
  // the same from a stream staged in LDS: entry q sits at sc[q - base], sv[q - base]
  __device__ __forceinline__ void load_lds(const int32_t* sc, const uint16_t* sv, int base, int p, int end) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int q = (p + i < end ? p + i : end - 1) - base;
      cc[i] = sc[q];
      vh[i] = sv[q];
    }
  }
  __device__ __forceinline__ void gather(const uint16_t* __restrict__ Bf, int64_t ldb) {
#pragma unroll
    for (int i = 0; i < U; ++i) bb[i].load(Bf + row_offset(cc[i], ldb));
  }
  // the same with staged hot rows (negative ids) at Hf
  __device__ __forceinline__ void gather_hot(const uint16_t* __restrict__ Bf, int64_t ldb,
                                             const uint16_t* __restrict__ Hf, int32_t hld) {
#pragma unroll
    for (int i = 0; i < U; ++i) bb[i].load(gather_addr<true>(Bf, ldb, Hf, hld, cc[i]));
  }
  // after gather(): fetch the next batch's column ids and values into n
  __device__ __forceinline__ void prefetch_next(Batch& n, const int32_t* __restrict__ col,
                                                const uint16_t* __restrict__ val, int p, int end) const {
    n.load_a(col, val, p + U, end);
  }
  __device__ __forceinline__ void advance(const Batch& n) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      cc[i] = n.cc[i];
      vh[i] = n.vh[i];
    }
  }
  // one step of a stream over [.., end) at batch start p (first = start of the stream, whose
  // column ids and values a pipelined stream loaded up front): loads of this batch (+ prefetch)
  template <bool PF>
  __device__ __forceinline__ void step_begin(Batch& n, const int32_t* __restrict__ col,
                                             const uint16_t* __restrict__ val, const uint16_t* __restrict__ Bf,
                                             int64_t ldb, int p, int end) {
    if constexpr (PF) {
      gather(Bf, ldb);
      prefetch_next(n, col, val, p, end);
    } else {
      load_a(col, val, p, end);
      gather(Bf, ldb);
    }
  }
  template <bool PF>
  __device__ __forceinline__ void step_end(const Batch& n) {
    if constexpr (PF) advance(n);
  }
};

// Accumulate entries [p0, p1) of one row into acc (U loads in flight).  Bf = B + feature offset
// (a valid column for lanes past K, whose sums are discarded).
template <int VEC, int U, bool NT, bool PF>
__device__ __forceinline__ void accumulate_row(const int32_t* __restrict__ col, const uint16_t* __restrict__ val,
                                               const uint16_t* __restrict__ Bf, int64_t ldb, int p0, int p1,
                                               float (&acc)[VEC]) {
  if (p0 >= p1) return;
  Batch<VEC, U, NT> b, n;
  if constexpr (PF) b.load_a(col, val, p0, p1);
  for (int p = p0; p < p1; p += U) {
    b.template step_begin<PF>(n, col, val, Bf, ldb, p, p1);
#pragma unroll
    for (int i = 0; i < U; ++i)
      if (p + i < p1) b.bb[i].fma(acc, h2f(b.vh[i]));
    b.template step_end<PF>(n);
  }
}

// ------------------------------------------------------------------------------------------------
// Streaming-hint bits of DevicePlan::streaming: non-temporal A-stream loads / C stores.
constexpr int kNtLoads = 1;
constexpr int kNtStores = 2;

// Staged A stream (LS): a lane group copies its task's column ids and values into LDS once, in
// whole 16-byte chunks from an 8-entry-aligned base (every chunk read by one load instruction, all
// loads issued before the first store; the plan's device block has 256 bytes of tail, so chunks
// ending past an array stay inside it), and its batches then read them from LDS.  The loads are
// non-temporal: each line is read exactly once, and the A stream then stays out of the caches that
// hold B rows.  Tasks hold <= kStageMax entries (the launcher checks DevicePlan::task_max).
constexpr int kStageMax = 256;
constexpr int kStageSpan = kStageMax + 8;
typedef int32_t int4_t __attribute__((ext_vector_type(4)));

template <int LPG>
__device__ __forceinline__ void stage_stream(const int32_t* __restrict__ col, const uint16_t* __restrict__ val,
                                             int nz_begin, int nz_end, int li, int32_t* sc, uint16_t* sv) {
  constexpr int CC = (kStageSpan / 4 + LPG - 1) / LPG;   // 4-entry column chunks per lane
  constexpr int VC = (kStageSpan / 8 + LPG - 1) / LPG;   // 8-entry value chunks per lane
  const int base = nz_begin & ~7;
  const int span = nz_end - base;
  const int clast = (span - 1) >> 2, vlast = (span - 1) >> 3;
  int4_t c[CC], v[VC];
#pragma unroll
  for (int k = 0; k < CC; ++k) {   // chunks past the span repeat the last one (same data, same slot)
    const int j = li + k * LPG <= clast ? li + k * LPG : clast;
    c[k] = load_stream<true>(reinterpret_cast<const int4_t*>(col + base) + j);
  }
#pragma unroll
  for (int k = 0; k < VC; ++k) {
    const int j = li + k * LPG <= vlast ? li + k * LPG : vlast;
    v[k] = load_stream<true>(reinterpret_cast<const int4_t*>(val + base) + j);
  }
#pragma unroll
  for (int k = 0; k < CC; ++k) {
    const int j = li + k * LPG <= clast ? li + k * LPG : clast;
    reinterpret_cast<int4_t*>(sc)[j] = c[k];
  }
#pragma unroll
  for (int k = 0; k < VC; ++k) {
    const int j = li + k * LPG <= vlast ? li + k * LPG : vlast;
    reinterpret_cast<int4_t*>(sv)[j] = v[k];
  }
}

// Column ids only (SDDMM has no values): same chunking and clamping as stage_stream.
template <int LPG>
__device__ __forceinline__ void stage_cols(const int32_t* __restrict__ col, int nz_begin, int nz_end, int li,
                                           int32_t* sc) {
  constexpr int CC = (kStageSpan / 4 + LPG - 1) / LPG;
  const int base = nz_begin & ~7;
  const int clast = (nz_end - base - 1) >> 2;
  int4_t c[CC];
#pragma unroll
  for (int k = 0; k < CC; ++k) {
    const int j = li + k * LPG <= clast ? li + k * LPG : clast;
    c[k] = load_stream<true>(reinterpret_cast<const int4_t*>(col + base) + j);
  }
#pragma unroll
  for (int k = 0; k < CC; ++k) {
    const int j = li + k * LPG <= clast ? li + k * LPG : clast;
    reinterpret_cast<int4_t*>(sc)[j] = c[k];
  }
}

// Static LDS of k_spmm_tasks<.., LPG, .., LS>: the row-pointer slices and, when staged, the column
// id and value slices (TasksLds; checked there).
constexpr size_t tasks_static_lds(int lpg, bool ls) {
  return (size_t)4 * (64 / lpg) * (kTaskRows + 1) * 4 + (ls ? (size_t)4 * (64 / lpg) * kStageSpan * 6 : 32);
}

// The task body's LDS, one block per (LPG, LS): the main and split parts of one launch run the body
// with different batch sizes, and arrays declared in the body would be allocated once per batch
// size (twice the LDS, half the occupancy).
template <int LPG, bool LS>
struct TasksLds {
  int rp[4][64 / LPG][kTaskRows + 1];
  alignas(16) int32_t col[LS ? 4 * (64 / LPG) * kStageSpan : 4];
  alignas(16) uint16_t val[LS ? 4 * (64 / LPG) * kStageSpan : 8];
};
template <int LPG, bool LS>
__device__ __forceinline__ TasksLds<LPG, LS>& tasks_lds() {
  __shared__ TasksLds<LPG, LS> s;
  return s;
}

// PF: pipelined stream (see Batch); the first batch's column ids and values are then loaded
// together with the row pointers, before the barrier.  LS: staged stream (see stage_stream).
// HOT: P.col is the hot-renumbered copy and negative ids gather from the staged rows P.hot_b
// (staged streams only).
template <int VEC, int LPG, int U, int NT, bool PF, bool LS, bool HOT = false>
__device__ __forceinline__ void spmm_tasks_run(const DevicePlan& P, int block, int nblocks,
                                               const uint16_t* __restrict__ B, int64_t ldb, int K,
                                               float* __restrict__ C, int64_t ldc, float* __restrict__ partial) {
  constexpr int GPW = 64 / LPG;
  constexpr bool NTL = (NT & kNtLoads) != 0;
  constexpr bool NTS = (NT & kNtStores) != 0;
  // row pointers of each lane group's task, preloaded once so a row flush never waits on a
  // dependent global load (tasks carry at most kTaskRows rows)
  TasksLds<LPG, LS>& lds = tasks_lds<LPG, LS>();
  auto& s_rp = lds.rp;
  int32_t* s_col = lds.col;
  uint16_t* s_val = lds.val;
  static_assert(!(LS && PF), "a staged stream is not pipelined");
  static_assert(!HOT || LS, "staged hot rows are read by the staged-stream kernel");
  static_assert(sizeof(TasksLds<LPG, LS>) == tasks_static_lds(LPG, LS),
                "tasks_static_lds must describe this kernel's LDS (the occupancy cap depends on it)");
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int grp = lane / LPG;
  const int li = lane % LPG;
  bool valid;
  const int task_id = residual_task(P, wave, grp, GPW, valid, block, nblocks);
  const Task t = valid ? P.tasks[task_id] : Task{0, 0, 0, 0};
  const int32_t* __restrict__ col = P.col;
  const uint16_t* __restrict__ val = P.val;
  int* rp = s_rp[wave][grp];
  if (valid && t.row_end >= 0) preload_rowptr<LPG>(P.rowptr, t.row_begin, t.row_end - t.row_begin, li, rp);
  Batch<VEC, U, NTL, (LPG == 2 || LPG == 4) ? LPG : 0> b, n;
  if constexpr (PF) {
    if (valid && t.nz_begin < t.nz_end) b.load_a(col, val, t.nz_begin, t.nz_end);
  }
  int32_t* sc = s_col + (LS ? (wave * GPW + grp) * kStageSpan : 0);
  uint16_t* sv = s_val + (LS ? (wave * GPW + grp) * kStageSpan : 0);
  const int sbase = t.nz_begin & ~7;
  if constexpr (LS) {
    if (valid && t.nz_begin < t.nz_end) stage_stream<LPG>(col, val, t.nz_begin, t.nz_end, li, sc, sv);
  }
  __syncthreads();
  if (!valid) return;

  const int f = blockIdx.y * (LPG * VEC) + li * VEC;
  const bool active = f < K;
  const uint16_t* __restrict__ Bf = B + (active ? f : 0);
  const uint16_t* __restrict__ Hf = HOT ? P.hot_b + (active ? f : 0) : nullptr;
  float acc[VEC];
  zero_acc(acc);
  // one batch: column ids and values (from LDS when staged) and its B gathers
  auto begin_batch = [&](int p, int end) {
    if constexpr (LS) {
      b.load_lds(sc, sv, sbase, p, end);
      if constexpr (HOT) b.gather_hot(Bf, ldb, Hf, P.hot_ld);
      else b.gather(Bf, ldb);
    } else {
      b.template step_begin<PF>(n, col, val, Bf, ldb, p, end);
    }
  };

  if (t.row_end < 0) {   // piece of a split row -> partial slot (re-read by the fixup: keep cached)
    for (int p = t.nz_begin; p < t.nz_end; p += U) {
      begin_batch(p, t.nz_end);
#pragma unroll
      for (int i = 0; i < U; ++i)
        if (p + i < t.nz_end) b.bb[i].fma(acc, h2f(b.vh[i]));
      b.template step_end<PF>(n);
    }
    if (active) store_vec<VEC>(partial + (int64_t)(~t.row_end) * K + f, acc);
    return;
  }
  // whole rows [row_begin, row_end): stream entries, flush a row when its end is crossed
  int r = 0;                       // row index relative to row_begin
  int rend = rp[1];
  for (int p = t.nz_begin; p < t.nz_end; p += U) {
    begin_batch(p, t.nz_end);
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (p + i < t.nz_end) {
        while (p + i >= rend) {
          if (active) store_vec<VEC, NTS>(C + (int64_t)(t.row_begin + r) * ldc + f, acc);
          zero_acc(acc);
          ++r;
          rend = rp[r + 1];
        }
        b.bb[i].fma(acc, h2f(b.vh[i]));
      }
    }
    b.template step_end<PF>(n);
  }
  for (; t.row_begin + r < t.row_end; ++r) {
    if (active) store_vec<VEC, NTS>(C + (int64_t)(t.row_begin + r) * ldc + f, acc);
    zero_acc(acc);
  }
}

// One launch for the main part (Pm, the first gm workgroups, into C) and the split part (Px, the
// rest, sub-row j into partial slot j); gm is a multiple of kXcds, so a split-part workgroup keeps
// its XCD (block mod kXcds).  One launch instead of two lets the split part start while the main
// part's last workgroups finish (same-box A/B on R-MAT 2^20: K = 128 0.706 -> 0.689 ms, K = 256
// 1.464 -> 1.420; the two parts' workgroups interleaved instead: 0.695 / 1.432, split part first
// 0.695 / 1.443; with 4 entries per batch, interleaved in chunks of kXcds workgroups: K = 128
// 0.614 -> 0.642 ms, K = 256 1.266 -> 1.290, K = 32 0.298 -> 0.316 -- the split part's per-XCD
// column classes keep their L2 hits only while the main part's gathers do not share the L2s).
// Without a split part, Px is unused and gm is the grid.
// The split part takes split_batch(...) entries per batch: with 16-byte loads, 8 in groups of >= 16
// lanes, where the main part takes 3 (its gathers miss the L2 about half the time and keep the
// memory busy, while the split part's mostly hit it and wait on latency), and 16 in groups of 8
// and 4 lanes, where the main part takes 8 and 32.  Same-box A/B, main / split entries per batch:
// R-MAT 2^20 K = 128 and 256: 4 / 4 0.610 / 1.267 ms, 3 / 8 0.597 / 1.244, 4 / 8 0.600 / 1.246,
// 2 / 8 0.597 / 1.253, 3 / 6 0.597 / 1.246, 3 / 12 0.609 / 1.265, 3 / 16 0.644 / 1.354, 6 / 4
// 0.619 / 1.281 (grid+hubs K = 128 1.144 / 1.151 (3 / 8) / 1.127 (3 / 12)); K = 64, R-MAT and
// grid+hubs: 8 / 8 0.450 / 0.588, 8 / 16 0.441 / 0.589, 4 / 8 0.454 / 0.639, 16 / 8 0.450 /
// 0.600, 12 / 16 0.447 / 0.593, 8 / 32 0.72 / 0.75; K = 32: 16 / 16 0.301 / 0.381, 32 / 16
// 0.300 / 0.367, 32 / 32 0.312 / 0.366, 16 / 32 0.309 / 0.381, 8 / 16 0.302 / 0.389, 48 / 16
// 0.435 / 0.450.
constexpr int split_batch(int vec, int lpg, int u) {
  return vec != 8 ? u : lpg >= 16 ? 8 : lpg == 8 || lpg == 4 ? 16 : u;
}
template <int VEC, int LPG, int U, int NT, bool PF, bool LS, bool HOT = false>
__global__ __launch_bounds__(256) void k_spmm_tasks(DevicePlan Pm, DevicePlan Px, int gm,
                                                    const uint16_t* __restrict__ B, int64_t ldb, int K,
                                                    float* __restrict__ C, int64_t ldc, float* __restrict__ partial) {
  constexpr int XU = split_batch(VEC, LPG, U);
  const int b = (int)blockIdx.x;
  if (b < gm) spmm_tasks_run<VEC, LPG, U, NT, PF, LS, HOT>(Pm, b, gm, B, ldb, K, C, ldc, partial);
  else spmm_tasks_run<VEC, LPG, XU, NT, PF, LS, HOT>(Px, b - gm, (int)gridDim.x - gm, B, ldb, K, partial, K, partial);
}

// C[row] = sum of a split row's partial slots, in slot order (deterministic), 4 slots in flight.
template <int VEC, int LPG>
__device__ __forceinline__ void fixup_narrow(const DevicePlan& P, int block, int K, float* __restrict__ C,
                                             int64_t ldc, const float* __restrict__ partial) {
  constexpr int GPW = 64 / LPG;
  constexpr int SU = 4;
  const int lane = threadIdx.x & 63;
  const int id = (block * 4 + (threadIdx.x >> 6)) * GPW + lane / LPG;
  if (id >= P.nfixups) return;
  const int f = blockIdx.y * (LPG * VEC) + (lane % LPG) * VEC;
  if (f >= K) return;
  const Fixup x = P.fixups[id];
  float acc[VEC];
  zero_acc(acc);
  for (int s = 0; s < x.slots; s += SU) {
    float v[SU][VEC];
#pragma unroll
    for (int u = 0; u < SU; ++u) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[u][i] = 0.f;
      if (s + u < x.slots) {
        const float* src = partial + (int64_t)P.slot_list[x.slot_begin + s + u] * K + f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[u][i] = src[i];
      }
    }
#pragma unroll
    for (int u = 0; u < SU; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] += v[u][i];
  }
  store_vec<VEC>(C + (int64_t)x.row * ldc + f, acc);
}

// Split rows with many slots: one workgroup per row.  Lane group g sums slots g, g + G, ... (in
// order), then the G group sums are combined by a fixed binary tree in LDS (deterministic).
template <int VEC, int LPG>
__device__ __forceinline__ void fixup_wide(const DevicePlan& P, int block, int K, float* __restrict__ C,
                                           int64_t ldc, const float* __restrict__ partial) {
  constexpr int G = 256 / LPG;
  __shared__ float red[G][LPG * VEC];
  const int g = threadIdx.x / LPG;
  const int li = threadIdx.x % LPG;
  const int f = blockIdx.y * (LPG * VEC) + li * VEC;
  const Fixup x = P.wfixups[block];
  float acc[VEC];
  zero_acc(acc);
  if (f < K) {
    for (int s = g; s < x.slots; s += G) {
      const float* src = partial + (int64_t)P.slot_list[x.slot_begin + s] * K + f;
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] += src[i];
    }
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) red[g][li * VEC + i] = acc[i];
  __syncthreads();
  for (int h = G / 2; h > 0; h >>= 1) {
    if (g < h)
#pragma unroll
      for (int i = 0; i < VEC; ++i) red[g][li * VEC + i] += red[g + h][li * VEC + i];
    __syncthreads();
  }
  if (g == 0 && f < K) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = red[0][li * VEC + i];
    store_vec<VEC>(C + (int64_t)x.row * ldc + f, acc);
  }
}

// Both kinds of split rows in one launch: blocks [0, nwfixups) take one wide row each, the rest
// the narrow rows, 4 waves x 64 / LPG lane groups per block (one launch instead of two: the
// narrow and wide sets write disjoint rows and run side by side).
template <int VEC, int LPG>
__global__ __launch_bounds__(256) void k_spmm_fixup(DevicePlan P, int K, float* __restrict__ C, int64_t ldc,
                                                    const float* __restrict__ partial) {
  if ((int)blockIdx.x < P.nwfixups) fixup_wide<VEC, LPG>(P, blockIdx.x, K, C, ldc, partial);
  else fixup_narrow<VEC, LPG>(P, (int)blockIdx.x - P.nwfixups, K, C, ldc, partial);
}

// ------------------------------------------------------------------------------------------------
// MFMA window kernel.  KC = features per workgroup (multiple of 16, <= 128); NT = MFMA n-tiles
// (16 features each) per wave = KC / 64 rounded up (template NTILE).
// MFMA 16x16x16 f16 operand layout (lane l, j = 0..3):
//   A: A[l % 16][4 * (l / 16) + j]      B: B[4 * (l / 16) + j][l % 16]
//   D: D[4 * (l / 16) + j][l % 16]
// Here A = the 16x16 tile (window row x tile column), B = gathered B rows (tile column x feature).
// Occupancy floor: the register budget of 6 waves per SIMD (the compiler settles at 5 otherwise;
// measured: 5 waves cost 6% on SBM K=128 and 4% at K=256, 0.963 vs 0.924 ms).
template <int VEC, int NTILE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6)))
void k_spmm_mfma_win(DevicePlan P, const uint16_t* __restrict__ B, int64_t ldb, int K, float* __restrict__ C,
                     int64_t ldc, int KC) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int KCP = KC + 4;   // fp32 output tile row stride
  const int KCB = KC + 8;   // fp16 staged-B row stride (keeps 16-byte alignment)
  float* otile = reinterpret_cast<float*>(smem);
  _Float16* bst = reinterpret_cast<_Float16*>(otile + 16 * KCP);

  const int wi = xcd_remap(blockIdx.x, gridDim.x, P.xcd_run);
  const MfmaWindow w = P.mwin[wi];
  const int fbase = blockIdx.y * KC;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int ntn = KC / 16;

  float4_t acc[NTILE];
#pragma unroll
  for (int j = 0; j < NTILE; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int t = w.tile_begin; t < w.tile_end; ++t) {
    // the tile's A fragment, loaded before the barrier so that it arrives under the B-row gathers
    // (same-box A/B on SBM, loaded after the staging barrier: K = 64 0.233 -> 0.226 ms, K = 128
    // 0.430 -> 0.425, K = 256 0.868 -> 0.858; non-temporal: no gain)
    const half4_t a = *reinterpret_cast<const half4_t*>(
        reinterpret_cast<const _Float16*>(P.tile_a) + (int64_t)t * 256 + (lane & 15) * 16 + 4 * (lane >> 4));
    __syncthreads();
    // stage the 16 gathered B rows (features [fbase, fbase + KC)) into LDS; empty column slots
    // and features past K are zeros, not gathered
    const int per_row = KC / VEC;
    for (int idx = threadIdx.x; idx < 16 * per_row; idx += 256) {
      const int k = idx / per_row;
      const int ff = (idx % per_row) * VEC;
      const int c = P.tile_cols[t * 16 + k];
      BFrag<VEC> b;
      if (c >= 0 && fbase + ff < K) b.load(B + row_offset(c, ldb) + fbase + ff);
      else b.zero();
      if constexpr (VEC == 8) *reinterpret_cast<half8_t*>(bst + k * KCB + ff) = b.v;
      else if constexpr (VEC == 4) *reinterpret_cast<half4_t*>(bst + k * KCB + ff) = b.v;
      else if constexpr (VEC == 2) *reinterpret_cast<half2_t*>(bst + k * KCB + ff) = b.v;
      else bst[k * KCB + ff] = b.v;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NTILE; ++j) {
      const int nt = wave + 4 * j;
      if (nt < ntn) {
        half4_t b;
#pragma unroll
        for (int i = 0; i < 4; ++i) b[i] = bst[(4 * (lane >> 4) + i) * KCB + nt * 16 + (lane & 15)];
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, acc[j], 0, 0, 0);
      }
    }
  }
  // 2:4 quads on the sparse MFMA (layout in DevicePlan): per chunk j of CW = min(KC, 64) features,
  // the quad's 64 B rows are staged row-major ([64][CW + 8] fp16, reusing the dense staging space;
  // only the features the chunk's n-tiles use: SBM K = 16 -1.4%, K = 32 -0.4% against whole
  // 64-feature rows); lane l's B operand is B[k][16 * wave + l % 16] for k = 8 (l / 16) + s (s < 8)
  // and 32 + 8 (l / 16) + s - 8 (s >= 8)
  if (P.win_quad) {
    const int CW = KC < 64 ? KC : 64;
    const int QS = CW + 8;   // staged row stride (fp16)
    const int qb = P.win_quad[wi], qe = P.win_quad[wi + 1];
    for (int q = qb; q < qe; ++q) {
      const half8_t a = reinterpret_cast<const half8_t*>(P.quad_a)[(int64_t)q * 64 + lane];
      const int idx = P.quad_idx[(int64_t)q * 64 + lane];
#pragma unroll
      for (int j = 0; j < NTILE; ++j) {
        __syncthreads();
        const int per_row = CW / VEC;
        for (int i2 = threadIdx.x; i2 < 64 * per_row; i2 += 256) {
          const int k = i2 / per_row;
          const int ff = (i2 % per_row) * VEC;
          const int c = P.quad_cols[(int64_t)q * 64 + k];
          const int f = fbase + 64 * j + ff;
          BFrag<VEC> b;
          if (c >= 0 && f < K) b.load(B + row_offset(c, ldb) + f);
          else b.zero();
          if constexpr (VEC == 8) *reinterpret_cast<half8_t*>(bst + k * QS + ff) = b.v;
          else if constexpr (VEC == 4) *reinterpret_cast<half4_t*>(bst + k * QS + ff) = b.v;
          else if constexpr (VEC == 2) *reinterpret_cast<half2_t*>(bst + k * QS + ff) = b.v;
          else bst[k * QS + ff] = b.v;
        }
        __syncthreads();
        if (wave + 4 * j < ntn) {
          half16_t b;
#pragma unroll
          for (int s2 = 0; s2 < 16; ++s2) {
            const int k = s2 < 8 ? 8 * (lane >> 4) + s2 : 32 + 8 * (lane >> 4) + (s2 - 8);
            b[s2] = bst[k * QS + wave * 16 + (lane & 15)];
          }
          acc[j] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(a, b, acc[j], idx, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NTILE; ++j) {
    const int nt = wave + 4 * j;
    if (nt < ntn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) otile[(4 * (lane >> 4) + i) * KCP + nt * 16 + (lane & 15)] = acc[j][i];
    }
  }
  __syncthreads();

  // residual rows of this window: a row group walks a row's entries, adds the MFMA share read
  // back from LDS (16-byte reads) and stores the finished row once
  const int gs = KC / VEC;         // threads per row group
  const int groups = 256 / gs;     // threads past groups * gs sit this phase out
  const int g = threadIdx.x / gs;
  const int ff = (threadIdx.x % gs) * VEC;
  const int f = fbase + ff;
  for (int rl = g; g < groups && rl < 16; rl += groups) {
    const int row = w.row0 + rl;
    if (row >= P.m) break;
    float racc[VEC];
    zero_acc(racc);
    // pipelined batches of 4 entries (same-box A/B on SBM against 8 unpipelined / 8 pipelined /
    // 4 unpipelined: K=64 0.230 vs 0.246 / 0.257 / 0.248 ms, K=128 0.430 vs 0.462 / 0.479 /
    // 0.468, K=256 0.909 vs 0.938 / 0.922 / 1.037)
    accumulate_row<VEC, 4, false, true>(P.col, P.val, B + (f < K ? f : 0), ldb, P.rowptr[row], P.rowptr[row + 1],
                                        racc);
    if (f >= K) continue;
    const float* src = otile + rl * KCP + ff;
    if constexpr (VEC == 8) {
      const float4_t lo = reinterpret_cast<const float4_t*>(src)[0];
      const float4_t hi = reinterpret_cast<const float4_t*>(src)[1];
      racc[0] += lo[0]; racc[1] += lo[1]; racc[2] += lo[2]; racc[3] += lo[3];
      racc[4] += hi[0]; racc[5] += hi[1]; racc[6] += hi[2]; racc[7] += hi[3];
    } else if constexpr (VEC == 4) {
      const float4_t v = reinterpret_cast<const float4_t*>(src)[0];
      racc[0] += v[0]; racc[1] += v[1]; racc[2] += v[2]; racc[3] += v[3];
    } else if constexpr (VEC == 2) {
      const float2_t v = reinterpret_cast<const float2_t*>(src)[0];
      racc[0] += v[0]; racc[1] += v[1];
    } else {
      racc[0] += src[0];
    }
    if ((P.streaming & 2) && K >= 8) store_vec<VEC, true>(C + (int64_t)row * ldc + f, racc);
    else store_vec<VEC, false>(C + (int64_t)row * ldc + f, racc);
  }
}

// ------------------------------------------------------------------------------------------------
// Sum v[i] (i < U) over the LPG lanes of a group, U <= LPG (powers of two), with LPG - 1 shuffles
// in total: log2(U) halving exchanges, after which lane li holds a partial sum of entry
// e = li / (LPG / U), then log2(LPG / U) xor steps finish it.  Returns that entry's sum.
// Two spellings of the same exchanges, chosen by the code the compiler makes of them (same-box
// A/B on R-MAT, 8 entries per batch): the recursive one for groups of >= 8 lanes (K=128
// 1.098 -> 1.032 ms, K=64 0.582 -> 0.549), the loop for 4-lane groups (K=32 0.476 -> 0.463).
// Exchanges over DPP row permutes instead of shuffles measured no faster (K=128 1.090 ms).
template <int LPG, int U, int OFF, int W>
__device__ __forceinline__ void rs_halve(float (&v)[U], int li) {
  if constexpr (W >= 1) {
    const bool upper = (li & OFF) != 0;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const float send = upper ? v[i] : v[i + W];
      const float keep = upper ? v[i + W] : v[i];
      v[i] = keep + __shfl_xor(send, OFF, 64);
    }
    rs_halve<LPG, U, OFF / 2, W / 2>(v, li);
  }
}
template <int OFF>
__device__ __forceinline__ float rs_finish(float v) {
  if constexpr (OFF >= 1) return rs_finish<OFF / 2>(v + __shfl_xor(v, OFF, 64));
  else return v;
}

template <int LPG, int U>
__device__ __forceinline__ float reduce_scatter(float (&v)[U], int li) {
  if constexpr (LPG >= 8) {
    rs_halve<LPG, U, LPG / 2, U / 2>(v, li);
    return rs_finish<LPG / (2 * U)>(v[0]);
  } else {
#pragma unroll
    for (int w = U / 2, off = LPG / 2; w >= 1; w >>= 1, off >>= 1) {
      const bool upper = (li & off) != 0;
#pragma unroll
      for (int i = 0; i < w; ++i) {
        const float send = upper ? v[i] : v[i + w];
        const float keep = upper ? v[i + w] : v[i];
        v[i] = keep + __shfl_xor(send, off, 64);
      }
    }
#pragma unroll
    for (int off = LPG / (2 * U); off >= 1; off >>= 1) v[0] += __shfl_xor(v[0], off, 64);
    return v[0];
  }
}

// Residual SDDMM: a lane group streams its task's entries U at a time (rows from the row pointers
// preloaded into LDS, as in k_spmm_tasks); each lane forms partial dot products over its VEC
// features of X[row] and Y[col] (X rows repeat across a row's entries and stay cached), and the
// U sums are finished by reduce_scatter.  Pieces of long rows carry a single row.  LS: the task's
// column ids are first staged in LDS (as in k_spmm_tasks), so batches do not re-read their cache
// lines through L2.  SPF: the next batch's column ids are loaded under the current gathers.  NTO:
// outputs are written with non-temporal stores, so they do not evict gathered Y rows from L2.
// acc: add to the outputs instead of writing them (a later feature pass of the same entries).
// HOT: P.col is the hot-renumbered copy and negative ids gather Y rows from the staged rows
// P.hot_b.
// Static LDS of k_sddmm_tasks<.., LPG, .., LS>: the row-pointer slices and, when staged, the
// column id slices (the arrays it declares; checked there).
constexpr size_t sddmm_static_lds(int lpg, bool ls) {
  return (size_t)4 * (64 / lpg) * (kTaskRows + 1) * 4 + (ls ? (size_t)4 * (64 / lpg) * kStageSpan * 4 : 16);
}

template <int VEC, int LPG, int U, bool LS, bool SPF = false, bool NTO = false, bool HOT = false>
__device__ __forceinline__ void sddmm_tasks_run(const DevicePlan& P, int block, int nblocks,
                                                const uint16_t* __restrict__ X, int64_t ldx,
                                                const uint16_t* __restrict__ Y, int64_t ldy, int K,
                                                float* __restrict__ out, int acc) {
  constexpr int GPW = 64 / LPG;
  constexpr int FPP = LPG * VEC;               // features per pass
  constexpr int UB = U < LPG ? U : LPG;        // entries per reduce_scatter batch
  __shared__ int s_rp[4][GPW][kTaskRows + 1];
  __shared__ __align__(16) int32_t s_col[LS ? 4 * GPW * kStageSpan : 4];
  static_assert(sizeof(s_rp) + sizeof(s_col) == sddmm_static_lds(LPG, LS),
                "sddmm_static_lds must describe this kernel's LDS (the occupancy cap depends on it)");
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int grp = lane / LPG;
  const int li = lane % LPG;
  bool valid;
  const int task_id = residual_task(P, wave, grp, GPW, valid, block, nblocks);
  const Task t = valid ? P.tasks[task_id] : Task{0, 0, 0, 0};
  const bool piece = t.row_end < 0;
  int* rp = s_rp[wave][grp];
  if (valid && !piece) preload_rowptr<LPG>(P.rowptr, t.row_begin, t.row_end - t.row_begin, li, rp);
  int32_t* sc = s_col + (LS ? (wave * GPW + grp) * kStageSpan : 0);
  const int sbase = t.nz_begin & ~7;
  if constexpr (LS) {
    if (valid && t.nz_begin < t.nz_end) stage_cols<LPG>(P.col, t.nz_begin, t.nz_end, li, sc);
  }
  // column ids of the batch at p (unconditional loads: padded slots repeat the last entry)
  auto load_cols = [&](int p, int (&cc)[U]) {
    if constexpr ((LPG == 2 || LPG == 4) && U % LPG == 0 && !LS) {
      // quad-shared column loads: lane j of the group loads entries p + j, p + j + LPG, ... and
      // the group exchanges them by DPP broadcasts, so a load instruction carries LPG times fewer
      // requests
      constexpr int R = U / LPG;
      int c[R];
#pragma unroll
      for (int k = 0; k < R; ++k) {
        const int q = p + k * LPG + li < t.nz_end ? p + k * LPG + li : t.nz_end - 1;
        c[k] = P.col[q];
      }
#pragma unroll
      for (int i = 0; i < U; ++i) cc[i] = group_bcast<LPG>(c[i / LPG], i % LPG);
    } else {
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int q = p + i < t.nz_end ? p + i : t.nz_end - 1;
        cc[i] = LS ? sc[q - sbase] : P.col[q];
      }
    }
  };
  // PF: the next batch's column ids are loaded while this batch's gathers are in flight; the
  // first batch's before the barrier
  constexpr bool PFC = SPF && !LS;
  int cn[U];
  if constexpr (PFC) {
    if (valid && t.nz_begin < t.nz_end) load_cols(t.nz_begin, cn);
  }
  __syncthreads();
  if (!valid) return;

  int r = 0;
  int rend = piece ? t.nz_end : rp[1];
  // with a single feature pass, the X fragment of the last row used carries over to the next
  // batch, so X is fetched once per row instead of once per batch
  const bool carry = K <= FPP;
  BFrag<VEC> xc;
  xc.zero();
  int xrow = -1;
  for (int p = t.nz_begin; p < t.nz_end; p += U) {
    int cc[U], rr[U];
    if constexpr (PFC) {
#pragma unroll
      for (int i = 0; i < U; ++i) cc[i] = cn[i];
    } else {
      load_cols(p, cc);
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const bool in = p + i < t.nz_end;
      if (in && !piece) {
        while (p + i >= rend) {
          ++r;
          rend = rp[r + 1];
        }
      }
      rr[i] = t.row_begin + r;
    }

    float s[U];
#pragma unroll
    for (int i = 0; i < U; ++i) s[i] = 0.f;
    for (int f0 = 0; f0 < K; f0 += FPP) {
      const int f = f0 + li * VEC;
      // all Y gathers first, unconditional so they issue back to back (lanes past K read features
      // [0, VEC) and padded slots repeat the last entry; both are discarded), then one X fetch per
      // distinct row of the chunk; the fragment each entry uses is selected in registers
      BFrag<VEC> x[U], y[U];
      const uint16_t* __restrict__ Yf = Y + (f < K ? f : 0);
      const uint16_t* __restrict__ Hf = HOT ? P.hot_b + (f < K ? f : 0) : nullptr;
#pragma unroll
      for (int i = 0; i < U; ++i) y[i].load(gather_addr<HOT>(Yf, ldy, Hf, P.hot_ld, cc[i]));
      if constexpr (PFC) {
        if (f0 == 0 && p + U < t.nz_end) load_cols(p + U, cn);
      }
      const bool reuse = carry && rr[0] == xrow;
      // X rows of 16-byte-load widths (>= 128 B per row slice) are read non-temporally: a row is
      // fetched once per task and carried in registers, so caching it only evicts gathered Y
      // rows (same-box A/B on R-MAT: K = 128 0.739 -> 0.728 ms, 0.836 -> 0.795 without hot rows,
      // K = 256 -0.5%); narrower rows share cache lines with the next row and stay cached (K = 32
      // / 64 with non-temporal X loads: +7.7% / +2.8%)
#pragma unroll
      for (int i = 0; i < U; ++i) {
        if (f < K && p + i < t.nz_end && (i == 0 ? !reuse : rr[i] != rr[i - 1])) {
          const uint16_t* xp = X + (int64_t)(P.sub_row ? P.sub_row[rr[i]] : rr[i]) * ldx + f;
          if constexpr (VEC == 8) x[i].load_nt(xp);
          else x[i].load(xp);
        } else {
          x[i].zero();
        }
      }
      BFrag<VEC> xe = reuse ? xc : x[0];
#pragma unroll
      for (int i = 0; i < U; ++i) {
        if (i > 0 && rr[i] != rr[i - 1]) xe = x[i];
        s[i] += xe.dot(y[i]);
      }
      if (carry) {
        xc = xe;
        xrow = rr[U - 1];
      }
    }
#pragma unroll
    for (int b = 0; b < U; b += UB) {
      float v[UB];
#pragma unroll
      for (int i = 0; i < UB; ++i) v[i] = s[b + i];
      const float sum = reduce_scatter<LPG, UB>(v, li);
      const int e = b + li / (LPG / UB);
      if (li % (LPG / UB) == 0 && p + e < t.nz_end) {
        const int q = p + e;
        float* o = &out[P.res_pos ? P.res_pos[q - P.res_off] : q - P.out_off];
        const float v = acc ? sum + *o : sum;
        if constexpr (NTO) __builtin_nontemporal_store(v, o);
        else *o = v;
      }
    }
  }
}

// Main part (Pm, the first gm workgroups, into out_m) and split part (Px, the rest, into out_x) in
// one launch, as k_spmm_tasks (gm a multiple of kXcds where a split part follows).
template <int VEC, int LPG, int U, bool LS, bool SPF = false, bool NTO = false, bool HOT = false>
__global__ __launch_bounds__(256) void k_sddmm_tasks(DevicePlan Pm, DevicePlan Px, int gm,
                                                     const uint16_t* __restrict__ X, int64_t ldx,
                                                     const uint16_t* __restrict__ Y, int64_t ldy, int K,
                                                     float* __restrict__ out_m, float* __restrict__ out_x, int acc) {
  const int b = (int)blockIdx.x;
  if (b < gm) sddmm_tasks_run<VEC, LPG, U, LS, SPF, NTO, HOT>(Pm, b, gm, X, ldx, Y, ldy, K, out_m, acc);
  else sddmm_tasks_run<VEC, LPG, U, LS, SPF, NTO, HOT>(Px, b - gm, (int)gridDim.x - gm, X, ldx, Y, ldy, K, out_x, acc);
}

// The split rows' outputs into place (one workgroup per merge task): contiguous stores, reads from
// the split part's buffer within the row's few runs.
template <bool NTO>
__global__ __launch_bounds__(256) void k_sddmm_merge(const MergeTask* __restrict__ tasks,
                                                     const int32_t* __restrict__ x_src,
                                                     const float* __restrict__ xbuf, float* __restrict__ out) {
  // every load of a thread issued before the first store (indices past the task read entry 0)
  constexpr int PER = kMergeTaskEntries / 256;
  const MergeTask t = tasks[blockIdx.x];
  int src[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = t.e_begin + (int)threadIdx.x + i * 256;
    src[i] = x_src[t.k_begin + (e < t.e_end ? e - t.e_begin : 0)];
  }
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = xbuf[src[i]];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = t.e_begin + (int)threadIdx.x + i * 256;
    if (e < t.e_end) {
      if constexpr (NTO) __builtin_nontemporal_store(v[i], out + e);
      else out[e] = v[i];
    }
  }
}

// SDDMM over dense tiles, one wave per tile (4 per workgroup).  With the 16x16x16 MFMA operand
// layout (see k_spmm_mfma_win), A = X[row0 + l % 16][k0 + 4 (l / 16) + j] and
// B = Y[col_{l % 16}][k0 + 4 (l / 16) + j]: each lane reads 4 consecutive features of one row.
// VEC4: K % 4 == 0 and 8-byte aligned rows (one 8-byte load per operand), else guarded scalars.
template <bool VEC4>
__global__ __launch_bounds__(256) void k_sddmm_mfma(DevicePlan P, const uint16_t* __restrict__ X, int64_t ldx,
                                                    const uint16_t* __restrict__ Y, int64_t ldy, int K,
                                                    float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = xcd_remap(blockIdx.x, gridDim.x, P.xcd_run) * 4 + (threadIdx.x >> 6);
  if (t >= P.ntiles) return;
  const int row = P.tile_row0[t] + (lane & 15);
  const int col = P.tile_cols[t * 16 + (lane & 15)];
  const bool xrow_ok = row < P.m;
  const bool ycol_ok = col >= 0;
  const uint16_t* xp = X + (int64_t)(xrow_ok ? row : 0) * ldx;
  const uint16_t* yp = Y + (int64_t)(ycol_ok ? col : 0) * ldy;
  float4_t acc{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += 16) {
    const int k = k0 + 4 * (lane >> 4);
    half4_t a{0, 0, 0, 0}, b{0, 0, 0, 0};
    if constexpr (VEC4) {
      if (k < K) {
        if (xrow_ok) a = *reinterpret_cast<const half4_t*>(xp + k);
        if (ycol_ok) b = *reinterpret_cast<const half4_t*>(yp + k);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (k + j < K) {
          if (xrow_ok) a[j] = __builtin_bit_cast(_Float16, xp[k + j]);
          if (ycol_ok) b[j] = __builtin_bit_cast(_Float16, yp[k + j]);
        }
      }
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, acc, 0, 0, 0);
  }
  // D[r][c] for r = 4 (l / 16) + j, c = l % 16: write the stored entries
  const int32_t* pos = P.tile_pos + (int64_t)t * 256;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = pos[(4 * (lane >> 4) + j) * 16 + (lane & 15)];
    if (e >= 0) out[e] = acc[j];
  }
}

// SDDMM over dense tiles with gfx950's v_mfma_f32_16x16x32_f16, K % 8 == 0 and 16-byte aligned
// rows: lane l supplies 8 consecutive features (one 16-byte load) of X row row0 + l % 16 as A and of
// Y row col_{l % 16} as B, for the feature group 8 (l / 16) of each 32-feature step.  A and B use
// the same lane/element -> feature assignment, so D[r][c] = X[r] . Y[c] whatever order the
// instruction sums its 32 products in.  The loads of up to 4 steps (128 features) are issued
// before their MFMAs.  Features past K read feature 0 and are zeroed in both operands.
__global__ __launch_bounds__(256) void k_sddmm_mfma32(DevicePlan P, const uint16_t* __restrict__ X, int64_t ldx,
                                                      const uint16_t* __restrict__ Y, int64_t ldy, int K,
                                                      float* __restrict__ out) {
  constexpr int SPC = 4;   // 32-feature steps per chunk of loads
  const int lane = threadIdx.x & 63;
  const int t = xcd_remap(blockIdx.x, gridDim.x, P.xcd_run) * 4 + (threadIdx.x >> 6);
  if (t >= P.ntiles) return;
  const int row = P.tile_row0[t] + (lane & 15);
  const int col = P.tile_cols[t * 16 + (lane & 15)];
  // rows past m and empty column slots read row 0: they only feed D rows / columns never stored
  const uint16_t* xp = X + (int64_t)(row < P.m ? row : 0) * ldx;   // ldx may exceed 2^31 (ldy may not)
  const uint16_t* yp = Y + row_offset(col >= 0 ? col : 0, ldy);
  const int fq = 8 * (lane >> 4);
  float4_t acc{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += 32 * SPC) {
    half8_t a[SPC], b[SPC];
#pragma unroll
    for (int i = 0; i < SPC; ++i) {
      const int k = k0 + 32 * i + fq;
      const int kk = k < K ? k : 0;
      a[i] = *reinterpret_cast<const half8_t*>(xp + kk);
      b[i] = *reinterpret_cast<const half8_t*>(yp + kk);
    }
#pragma unroll
    for (int i = 0; i < SPC; ++i) {
      const bool in = k0 + 32 * i + fq < K;
      const half8_t z{0, 0, 0, 0, 0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(in ? a[i] : z, in ? b[i] : z, acc, 0, 0, 0);
    }
  }
  const int32_t* pos = P.tile_pos + (int64_t)t * 256;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = pos[(4 * (lane >> 4) + j) * 16 + (lane & 15)];
    if (e >= 0) out[e] = acc[j];
  }
}


// LDS of one CU on gfx950.  The residual task kernel can be held to fewer workgroups per CU than
// its registers allow by giving each workgroup unused dynamic LDS.
constexpr int kLdsPerCu = 160 * 1024;

// Dynamic LDS that lets at most `waves` 256-thread workgroups (= waves per SIMD) share a CU, given
// the kernel's static LDS; 0 = uncapped.  waves >= 2 keeps a workgroup's LDS under the 64 KB
// limit.  The 256-byte margin absorbs alignment of the static arrays.
inline size_t occupancy_pad(size_t lds_static, int waves) {
  if (waves <= 0) return 0;
  const size_t want = (size_t)kLdsPerCu / (size_t)(waves + 1) + 256;
  return want > lds_static ? want - lds_static : 0;
}

// The plan as the residual kernels see its split part: sub-rows for rows, the per-XCD queues for
// tasks (workgroup i takes queue i mod kXcds).
DevicePlan split_view(const DevicePlan& p) {
  DevicePlan v = p;
  v.rowptr = p.x_rowptr;
  v.tasks = p.x_tasks;
  v.ntasks = p.x_ntasks;
  v.task_max = p.x_task_max;
  v.xcd_queues = 1;
  v.sub_row = p.x_sub_row;
  v.res_pos = p.x_pos;          // SDDMM: the split entries' output indices (follow the main part)
  v.res_off = (int32_t)p.nnz_csr;
  return v;
}

template <int VEC, int LPG, int U, int NT, bool PF, bool LS, bool HOT = false>
void launch_tasks(dim3 grid, int gm, int waves, hipStream_t s, const DevicePlan& p, const DevicePlan& x,
                  const uint16_t* B, int64_t ldb, int K, float* C, int64_t ldc, float* partial) {
  hipLaunchKernelGGL((k_spmm_tasks<VEC, LPG, U, NT, PF, LS, HOT>), grid, dim3(256),
                     occupancy_pad(tasks_static_lds(LPG, LS), waves), s, p, x, gm, B, ldb, K, C, ldc, partial);
}

// Staged hot rows: dst[r][0, K) = B[rows[r]][0, K) for r < nhot, 16 bytes per thread (K % 8 == 0,
// 16-byte aligned rows).
__global__ __launch_bounds__(256) void k_stage_hot_rows(const uint16_t* __restrict__ B, int64_t ldb, int K,
                                                        const int32_t* __restrict__ rows, int32_t nhot,
                                                        uint16_t* __restrict__ dst) {
  const int chunks = K >> 3;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)nhot * chunks) return;
  const int r = (int)(t / chunks), c = (int)(t - (int64_t)r * chunks);
  const int4_t v = *reinterpret_cast<const int4_t*>(B + row_offset(rows[r], ldb) + c * 8);
  *reinterpret_cast<int4_t*>(dst + (int64_t)r * K + c * 8) = v;
}

// Copies the plan's hot rows of B (K features) into hot and returns the view whose task kernels
// read the renumbered columns and the staged rows.
DevicePlan hot_view(const DevicePlan& p, const uint16_t* B, int64_t ldb, int K, uint16_t* hot, hipStream_t s) {
  const int64_t threads = (int64_t)p.nhot * (K >> 3);
  hipLaunchKernelGGL(k_stage_hot_rows, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, B, ldb, K,
                     p.hot_rows, p.nhot, hot);
  DevicePlan v = p;
  v.col = p.hot_col;
  v.hot_b = hot;
  v.hot_ld = K;
  return v;
}

int lanes_for(int K, int vec) {
  const int need = (K + vec - 1) / vec;
  int l = 1;
  while (l < need && l < 64) l <<= 1;
  return l;
}

// Narrow loads of a width just past a power of two leave most lanes of a wide group idle: the
// group width (>= 16 lanes) with the fewest lane slots over all feature passes (ties to fewer
// passes), taken when it saves at least a fifth of the slots of `lpg` lanes.
int fewer_lane_slots(int K, int vec, int lpg) {
  const int slots0 = (K + lpg * vec - 1) / (lpg * vec) * lpg;
  int best = lpg, best_slots = slots0;
  for (int l = lpg / 2; l >= 16; l >>= 1) {
    const int slots = (K + l * vec - 1) / (l * vec) * l;
    if (slots < best_slots) best = l, best_slots = slots;
  }
  return best_slots * 5 <= slots0 * 4 ? best : lpg;
}

template <int VEC>
hipError_t launch_spmm_vec(const DevicePlan& p, const uint16_t* B, int64_t ldb, int K, float* C, int64_t ldc,
                           float* partial, uint16_t* hot, hipStream_t s, hipEvent_t* ev) {
  if (ev) (void)hipEventRecord(ev[0], s);
  int lpg = lanes_for(K, VEC);
  // a plan may ask for fewer lanes per group: several feature passes, each gathering a narrower
  // slice of B (smaller working set per pass)
  while (p.feature_lanes > 0 && lpg > p.feature_lanes && lpg > 1) lpg >>= 1;
  // (same-box A/B on R-MAT: K=66 2.25 ms in one pass of 64 lanes -> 1.93 in three of 16, K=130
  // 4.59 -> 3.21, K=65 3.14 -> 2.42, K=81 3.20 -> 2.78, K=33 1.47 -> 1.35; grid+hubs K=66 1.99 ->
  // 2.07, K=33 1.41 -> 1.46.  K=97, an eighth fewer slots in seven passes: 3.25 -> 3.33)
  if (p.feature_lanes <= 0 && VEC <= 2) lpg = fewer_lane_slots(K, VEC, lpg);
  // passes of at most 128 features for 16-byte loads: each pass gathers 256-byte slices of B
  // rows, twice as many of which fit an XCD's L2 as whole 512-byte rows (R-MAT 2^20, K = 256:
  // 1.730 ms in one pass of 32 lanes, 1.522 in two of 16, 1.837 in four of 8; K = 128 in two
  // passes of 64 features: 0.748 -> 0.910)
  if (p.feature_lanes <= 0 && VEC == 8 && lpg > 16) lpg = 16;
  // at least 4 lanes, whose column/value loads are shared, also where K < 4 leaves lanes idle
  // (same-box A/B: R-MAT K=1 0.316 -> 0.183 ms, K=2 0.255 -> 0.201; grid+hubs K=1 0.201 -> 0.122,
  // K=2 0.237 -> 0.175; 8 lanes at K=3: R-MAT 0.214 -> 0.258)
  if (p.feature_lanes <= 0 && lpg < 4) lpg = 4;
  const int fpp = lpg * VEC;
  const int passes = (K + fpp - 1) / fpp;
  // staged hot rows for the staged-stream kernel of 16-lane groups (256-byte gathers); the window
  // kernel keeps reading B through the plain column ids
  const bool hot_on = VEC == 8 && lpg == 16 && hot != nullptr && hot_buffer_bytes(p, K) > 0 &&
                      p.task_max <= kStageMax && p.stage >= 0 &&
                      (p.x_ntasks == 0 || p.x_task_max <= kStageMax);
  const DevicePlan tp = hot_on ? hot_view(p, B, ldb, K, hot, s) : p;
  // the main part writes C; the split part (XCD column split) writes sub-row j to partial slot j;
  // both in one launch (see k_spmm_tasks)
  const DevicePlan xv = split_view(tp);
  auto run_tasks = [&](const DevicePlan& p, const DevicePlan& x) {
    const int gpw = 64 / lpg;
    const int gx = x.ntasks > 0 ? residual_grid(x, gpw) : 0;   // a multiple of kXcds
    const int gm = p.ntasks <= 0 ? 0 : gx > 0 ? (residual_grid(p, gpw) + kXcds - 1) / kXcds * kXcds : residual_grid(p, gpw);
    if (gm + gx == 0) return;
    dim3 grid(gm + gx, passes);
    // entries per batch: 8 for narrow groups (K <= 64: short gathers, many in flight pay), 4 for
    // groups of >= 16 lanes (same-box A/B on R-MAT 2^20 with the staged stream and staged hot
    // rows, 2 / 3 / 4 / 6 / 8 entries: K=128 0.687 / 0.631 / 0.612 / 0.611 / 0.616 ms, K=256
    // 1.416 / 1.298 / 1.265 / 1.261 / 1.269, K=96 0.610 / - / 0.526 / - / 0.536; grid+hubs K=128
    // 1.142 / - / 1.145 / - / 1.142; before the staged stream 2 had measured best: K=128 1.12 ms
    // vs 1.24 with 8; K=32 0.54 ms with 8 vs 1.07 with 2); 16 for 4-lane groups of 16-byte loads
    // (K = 32: R-MAT 0.311 -> 0.303 ms, grid+hubs 0.393 -> 0.383; 8-lane groups at K = 64 gain
    // 0.6% on R-MAT and lose 2% on grid+hubs with 16, and keep 8).  With 16-byte loads the two
    // parts then took batches of their own (split_batch): the main part 3 at >= 16 lanes, 8 at 8
    // lanes and 32 at 4 lanes, the split part 8, 16 and 16
    // pipelined stream for narrow groups with long tasks (same-box A/B: R-MAT K=32/64
    // -9%/-12%; K=128 +8%, grid+hubs K=32 (32-entry tasks, 4 lanes) +6%), and for 8-lane groups
    // whatever the task length (grid+hubs K=64 0.620 -> 0.582 ms, K=8 0.251 -> 0.238)
    const bool pf = lpg <= 8 && (p.task_nnz >= 64 || lpg == 8);
    // staged A stream for 16-lane groups (K = 65..128; same-box A/B on R-MAT K=128: 1.118 ->
    // 0.975 ms, non-temporal staging loads 1% better than plain ones; K=256 +4%, not staged).
    // Its 27 KB of LDS per workgroup hold it at 5 waves per SIMD; that is not where the gain
    // comes from (the unstaged kernel forced to 5 waves takes 1.27 ms), and staging 128 entries
    // at a time to reach 8 waves measured 1.02 ms.
    const bool ls = p.task_max <= kStageMax && p.stage >= 0 && (x.ntasks <= 0 || x.task_max <= kStageMax);
    // occupancy: lane groups of <= 8 lanes (K <= 64) run 8 entries per batch and are held to 2 waves
    // per SIMD (same-box A/B at 7/6/5/4/3/2 waves: grid+hubs K=32 0.426 ... 0.395 / 0.389 ms,
    // R-MAT K=32 0.495 -> 0.420, K=64 0.579 -> 0.519, K=16 0.456 -> 0.400); wider groups are not
    // capped (R-MAT K=128 with 2 entries per batch at 5 / 4 / 3 waves: 0.970 / 0.985 / 1.147 ms,
    // K=256 at 8 / 3 waves: 2.24 / 3.49; with 4 entries per batch, capped at 3 or 4 waves: slower
    // than uncapped at K = 128 and 256)
    // (2-byte loads, used for K <= 8 and odd widths, stay uncapped: R-MAT K=8 0.293 ms uncapped,
    // 0.326 at 2 waves)
    // (4-byte loads in 8-lane groups, K = 10 and 14: 4 waves; R-MAT K=10 0.358 ms uncapped, 0.346
    // at 4 waves, 0.396 at 2)
    const int waves = p.occupancy > 0 ? p.occupancy : p.occupancy < 0 ? 0
                    : lpg <= 8 ? (VEC >= 4 ? 2 : VEC == 2 ? 4 : 0) : 0;
    // non-temporal C stores only where a row is at least 32 bytes (K >= 8): shorter rows lose
    // the L2's write combining (same-box A/B on grid+hubs: K=4 0.226 ms plain vs 0.246 streamed,
    // K=1 0.201 vs 0.208; K=8 0.292 plain vs 0.242 streamed, R-MAT K=16 0.341 vs 0.320)
    const int streaming = K >= 8 ? (p.streaming & 3) : (p.streaming & 1);
#define TRS_TASKS_NT(L, U, PF, LS, ...)                                                                   \
    switch (streaming) {                                                                                  \
      case 0: launch_tasks<VEC, L, U, 0, PF, LS, ##__VA_ARGS__>(grid, gm, waves, s, p, x, B, ldb, K, C, ldc, partial); break;   \
      case 1: launch_tasks<VEC, L, U, 1, PF, LS, ##__VA_ARGS__>(grid, gm, waves, s, p, x, B, ldb, K, C, ldc, partial); break;   \
      case 2: launch_tasks<VEC, L, U, 2, PF, LS, ##__VA_ARGS__>(grid, gm, waves, s, p, x, B, ldb, K, C, ldc, partial); break;   \
      default: launch_tasks<VEC, L, U, 3, PF, LS, ##__VA_ARGS__>(grid, gm, waves, s, p, x, B, ldb, K, C, ldc, partial); break;  \
    }
#define TRS_TASKS(L)                                                                                      \
  case L: {                                                                                               \
    constexpr int U = L >= 16 ? (VEC == 8 ? 3 : 4) : (L == 4 && VEC == 8) ? 32 : 8;                     \
    if constexpr (L <= 8) {                                                                               \
      if (pf) { TRS_TASKS_NT(L, U, true, false) } else { TRS_TASKS_NT(L, U, false, false) }               \
    } else if constexpr (L == 16) {                                                                       \
      if (VEC == 8 && p.hot_b != nullptr) { TRS_TASKS_NT(L, U, false, true, VEC == 8) }                   \
      else if (ls) { TRS_TASKS_NT(L, U, false, true) } else { TRS_TASKS_NT(L, U, false, false) }          \
    } else {                                                                                              \
      TRS_TASKS_NT(L, U, false, false)                                                                    \
    }                                                                                                     \
    break;                                                                                                \
  }
    switch (lpg) { TRS_TASKS(1) TRS_TASKS(2) TRS_TASKS(4) TRS_TASKS(8) TRS_TASKS(16) TRS_TASKS(32) TRS_TASKS(64) }
#undef TRS_TASKS
#undef TRS_TASKS_NT
  };
  if (tp.split_dispatch && tp.ntasks > 0 && xv.ntasks > 0) {
    // profiling layout: the main part, then the split part, as launches of their own
    DevicePlan main_only = xv, split_only = tp;
    main_only.ntasks = 0;
    split_only.ntasks = 0;
    run_tasks(tp, main_only);
    run_tasks(split_only, xv);
  } else {
    run_tasks(tp, xv);
  }
  if (ev) (void)hipEventRecord(ev[1], s);
  if (p.nmwin > 0) {
    const int kc16 = ((K + 15) / 16) * 16;
    // at most 128 features per workgroup: wider B slices in flight per window cost L2 capacity
    // (SBM 1M, K = 256: 0.912 ms with 256 features per workgroup, 0.871 with two of 128)
    const int KC = kc16 < 128 ? kc16 : 128;
    dim3 grid(p.nmwin, (K + KC - 1) / KC);
    // staging space: 16 dense-tile B rows of KC features, or a quad's 64 rows of min(KC, 64)
    const int cw = KC < 64 ? KC : 64;
    const size_t stage = std::max<size_t>((size_t)16 * (KC + 8), p.nquads > 0 ? (size_t)64 * (cw + 8) : 0);
    const size_t shm = (size_t)16 * (KC + 4) * 4 + stage * 2;
    if (KC <= 64) hipLaunchKernelGGL((k_spmm_mfma_win<VEC, 1>), grid, dim3(256), shm, s, p, B, ldb, K, C, ldc, KC);
    else hipLaunchKernelGGL((k_spmm_mfma_win<VEC, 2>), grid, dim3(256), shm, s, p, B, ldb, K, C, ldc, KC);
  }
  if (ev) (void)hipEventRecord(ev[2], s);
  if (p.nfixups > 0 || p.nwfixups > 0) {
    const int gpb = 4 * (64 / lpg);
    dim3 grid(p.nwfixups + (p.nfixups + gpb - 1) / gpb, passes);
#define TRS_FIX(L) case L: hipLaunchKernelGGL((k_spmm_fixup<VEC, L>), grid, dim3(256), 0, s, p, K, C, ldc, partial); break;
    switch (lpg) { TRS_FIX(1) TRS_FIX(2) TRS_FIX(4) TRS_FIX(8) TRS_FIX(16) TRS_FIX(32) TRS_FIX(64) }
#undef TRS_FIX
  }
  if (ev) (void)hipEventRecord(ev[3], s);
  return hipGetLastError();
}

template <int VEC>
hipError_t launch_sddmm_vec(const DevicePlan& p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy,
                            int K, float* out, uint16_t* hot, float* xbuf, hipStream_t s, hipEvent_t* ev) {
  if (ev) (void)hipEventRecord(ev[0], s);
  // staged hot Y rows (all K features, once per call) for the passes run by 16-lane groups
  const bool hot_on = VEC == 8 && hot != nullptr && hot_buffer_bytes(p, K) > 0;
  const DevicePlan hp = hot_on ? hot_view(p, Y, ldy, K, hot, s) : p;
  // the split part writes its own buffer (then merged) where the workspace holds one
  bool merge_on = p.x_ntasks > 0 && xbuf != nullptr && merge_buffer_bytes(p, K) > 0;
  // feature passes of at most 128 features for 16-byte loads, each over all entries, the later
  // ones adding to the outputs: 256-byte slices of Y rows keep twice as many rows in an XCD's L2
  // as whole 512-byte rows, for one extra read and write of each output per pass (R-MAT 2^20
  // pattern, K = 256: 1.793 ms in one pass of 32 lanes, 1.742 in two of 16)
  const int fpass = VEC == 8 && K > 128 && p.feature_lanes <= 0 ? 128 : K;
  for (int f0 = 0; f0 < K; f0 += fpass) {
    const int Kp = K - f0 < fpass ? K - f0 : fpass;
    const uint16_t* Xp = X + f0;
    const uint16_t* Yp = Y + f0;
    const int acc = f0 > 0 ? 1 : 0;
    DevicePlan pp = p;
    int lpg = lanes_for(Kp, VEC);
    // fewer lanes than features: the kernel loops over feature chunks per batch (no second walk
    // of the entries), so narrow loads take the group width with the fewest lane slots (same-box
    // A/B on R-MAT: K=66 1.49 ms with 64 lanes -> 0.91 with 16, K=82 1.50 -> 0.99, K=130 2.00 ->
    // 1.72, K=33 1.40 -> 0.73, K=65 1.87 -> 1.20)
    while (p.feature_lanes > 0 && lpg > p.feature_lanes && lpg > 1) lpg >>= 1;
    if (p.feature_lanes <= 0 && VEC <= 2) lpg = fewer_lane_slots(Kp, VEC, lpg);
    // at least 8 lanes, so that a group writes 8 consecutive sums (32 bytes) per store and the
    // outputs stream; lanes past K add zeros (R-MAT K=4 0.329 -> 0.258 ms, K=2 0.327 -> 0.259,
    // K=1 0.467 -> 0.260)
    if (p.feature_lanes <= 0 && lpg < 8) lpg = 8;
    if (hot_on && lpg == 16) {
      pp = hp;
      pp.hot_b = hot + f0;
    }
    // the main part (into out) and the split part (XCD column split, into xout) in one launch
    auto run_tasks = [&](const DevicePlan& p, float* out, const DevicePlan& x, float* xout) {
    const int gpw = 64 / lpg;
    const int gx = x.ntasks > 0 ? residual_grid(x, gpw) : 0;   // a multiple of kXcds
    const int gm = p.ntasks <= 0 ? 0 : gx > 0 ? (residual_grid(p, gpw) + kXcds - 1) / kXcds * kXcds : residual_grid(p, gpw);
    if (gm + gx == 0) return;
    dim3 grid(gm + gx);
    // column ids staged in LDS for 16-lane groups (K = 65..128; same-box A/B on R-MAT K=128:
    // 1.140 -> 1.112 ms; K=256 +1%, not staged); groups of <= 8 lanes load the next batch's
    // column ids while the current batch's gathers are in flight (K=32 0.429 -> 0.416 ms, K=8
    // -1%; 32-lane groups +1%, not pipelined); outputs written with non-temporal stores unless
    // the plan asks for plain ones, where a group writes 8 consecutive sums (32 bytes) per store
    // (same-box A/B on R-MAT: K=8 0.329 -> 0.264 ms, K=32 0.423 -> 0.394, K=64 -1.5%, K=128 -1%;
    // 16-byte runs, as 4-lane groups write at K=16, lose: 0.418 -> 0.469)
    const bool ls = p.task_max <= kStageMax && p.stage >= 0 && (x.ntasks <= 0 || x.task_max <= kStageMax);
    const bool nto = (p.streaming & 2) != 0;
    // occupancy: uncapped unless the plan asks (option occupancy: waves per SIMD, held by unused
    // dynamic LDS)
    const int waves = p.occupancy > 0 ? p.occupancy : 0;
#define TRS_SD_LAUNCH(VV, LL, UU, LSV, ...)                                                               \
  hipLaunchKernelGGL((k_sddmm_tasks<VV, LL, UU, LSV, ##__VA_ARGS__>), grid, dim3(256),                    \
                     occupancy_pad(sddmm_static_lds(LL, LSV), waves), s, p, x, gm, Xp, ldx, Yp, ldy, Kp, out, xout, acc)
#define TRS_SD_U(L, U)                                                                                     \
    constexpr bool nt_ok = (U < L ? U : L) >= 8;                                                           \
    if constexpr (L == 16) {                                                                               \
      if (VEC == 8 && p.hot_b != nullptr) {                                                                \
        if (ls) {                                                                                          \
          if (nt_ok && nto) TRS_SD_LAUNCH(VEC, L, U, true, false, nt_ok, VEC == 8);                        \
          else TRS_SD_LAUNCH(VEC, L, U, true, false, false, VEC == 8);                                     \
        } else {                                                                                           \
          if (nt_ok && nto) TRS_SD_LAUNCH(VEC, L, U, false, false, nt_ok, VEC == 8);                       \
          else TRS_SD_LAUNCH(VEC, L, U, false, false, false, VEC == 8);                                    \
        }                                                                                                  \
        break;                                                                                             \
      }                                                                                                    \
      if (ls) {                                                                                            \
        if (nt_ok && nto) TRS_SD_LAUNCH(VEC, L, U, true, false, nt_ok);                                    \
        else TRS_SD_LAUNCH(VEC, L, U, true);                                                               \
        break;                                                                                             \
      }                                                                                                    \
    }                                                                                                      \
    if (nt_ok && nto) TRS_SD_LAUNCH(VEC, L, U, false, (L <= 8), nt_ok);                                    \
    else TRS_SD_LAUNCH(VEC, L, U, false, (L <= 8));
    // entries in flight per lane group: 4 where a 16-lane group's 16-byte loads cover 128 features,
    // 8 elsewhere (same-box A/B on the R-MAT 2^20 pattern, 8 -> 4: K = 128 0.726 -> 0.705 ms, K = 256
    // (two passes of 128) 1.544 -> 1.482; K = 96 0.689 -> 0.720, K = 32 0.380 -> 0.488)
    const bool u4 = p.sddmm_unroll == 4 || (p.sddmm_unroll == 0 && VEC == 8 && lpg == 16 && Kp == 128);
#define TRS_SD(L)                                                                                          \
  case L:                                                                                                  \
    if (u4) {                                                                                              \
      TRS_SD_U(L, 4)                                                                                       \
    } else {                                                                                               \
      TRS_SD_U(L, 8)                                                                                       \
    }                                                                                                      \
    break;
    switch (lpg) { TRS_SD(1) TRS_SD(2) TRS_SD(4) TRS_SD(8) TRS_SD(16) TRS_SD(32) TRS_SD(64) }
#undef TRS_SD
#undef TRS_SD_U
#undef TRS_SD_LAUNCH
    };
    DevicePlan none = pp;
    none.ntasks = 0;
    if (lpg <= 8 && p.nnarrow_tasks > 0) {
      // lane groups of <= 8 lanes: the unsplit layout of every row in pieces of S entries, every
      // output written in place (no split part, nothing to merge)
      DevicePlan v = pp;
      v.tasks = p.narrow_tasks;
      v.ntasks = p.nnarrow_tasks;
      run_tasks(v, out, none, out);
      merge_on = false;
    } else if (merge_on) {
      // the split part into its own buffer, merged below
      DevicePlan v = split_view(pp);
      v.res_pos = nullptr;
      v.out_off = (int32_t)p.nnz_csr;
      if (p.split_dispatch && pp.ntasks > 0) {
        // profiling layout: main part and split part as launches of their own
        DevicePlan vnone = v;
        vnone.ntasks = 0;
        run_tasks(pp, out, vnone, xbuf);
        run_tasks(none, out, v, xbuf);
      } else {
        run_tasks(pp, out, v, xbuf);
      }
    } else if (p.x_ntasks > 0 && (K < kSddmmSplitMinK || hot_on)) {
      // written in place, the split part's scattered outputs cost more than it saves below
      // kSddmmSplitMinK, and wherever hot rows are staged (R-MAT 2^20 K = 128 0.777 vs 0.773 ms
      // unsplit, K = 256 1.693 vs 1.570): the unsplit layout of every row
      DevicePlan v = pp;
      v.tasks = p.full_tasks;
      v.ntasks = p.nfull_tasks;
      run_tasks(v, out, none, out);
    } else if (p.split_dispatch && p.x_ntasks > 0 && pp.ntasks > 0) {
      DevicePlan v = split_view(pp), vnone = split_view(pp);
      vnone.ntasks = 0;
      run_tasks(pp, out, vnone, out);
      run_tasks(none, out, v, out);
    } else {
      run_tasks(pp, out, p.x_ntasks > 0 ? split_view(pp) : none, out);
    }
  }
  if (merge_on) {
    if (p.streaming & 2) hipLaunchKernelGGL(k_sddmm_merge<true>, dim3(p.nmerge), dim3(256), 0, s, p.merge, p.x_src, xbuf, out);
    else hipLaunchKernelGGL(k_sddmm_merge<false>, dim3(p.nmerge), dim3(256), 0, s, p.merge, p.x_src, xbuf, out);
  }
  if (ev) (void)hipEventRecord(ev[1], s);
  if (p.ntiles > 0 && p.tile_pos) {
    const bool v4 = K % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(Y) & 7) == 0;
    const bool v8 = K % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && aligned16(X) && aligned16(Y);
    dim3 grid((p.ntiles + 3) / 4);
    // 16x16x32 with 16-byte loads issued ahead (same-box A/B on SBM 1M: K=128 0.174 -> 0.116 ms,
    // K=256 0.314 -> 0.205 ms; K=32 unchanged)
    if (v8) hipLaunchKernelGGL(k_sddmm_mfma32, grid, dim3(256), 0, s, p, X, ldx, Y, ldy, K, out);
    else if (v4) hipLaunchKernelGGL((k_sddmm_mfma<true>), grid, dim3(256), 0, s, p, X, ldx, Y, ldy, K, out);
    else hipLaunchKernelGGL((k_sddmm_mfma<false>), grid, dim3(256), 0, s, p, X, ldx, Y, ldy, K, out);
  }
  if (ev) (void)hipEventRecord(ev[2], s);
  return hipGetLastError();
}

#endif  // TRS_KERNEL_PART > 0

// ------------------------------------------------------------------------------------------------
// Device-side plan lowering (part 0 only).
#if TRS_KERNEL_PART == 0

// One workgroup per tile, one thread per (row, column) slot: binary search of the column in the
// CSR row (columns ascending) and mark the entry; an entry counts when its flag was clear.
__global__ __launch_bounds__(256) void k_mark_tile_entries(const TileEntries* __restrict__ tiles, int32_t m,
                                                           const int32_t* __restrict__ rowptr,
                                                           const int32_t* __restrict__ col,
                                                           uint32_t* __restrict__ flag_words,
                                                           uint32_t* __restrict__ marked,
                                                           int32_t* __restrict__ tile_pos) {
  const TileEntries& t = tiles[blockIdx.x];
  const int r = threadIdx.x >> 4, k = threadIdx.x & 15;
  const int row = t.row0 + r;
  if (!((t.present[r >> 2] >> ((r & 3) * 16 + k)) & 1) || row >= m) return;
  const int32_t c = t.cols[k];
  int lo = rowptr[row], hi = rowptr[row + 1];
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (col[mid] < c) lo = mid + 1;
    else hi = mid;
  }
  if (lo < rowptr[row + 1] && col[lo] == c) {
    const uint32_t bit = 1u << ((lo & 3) * 8);
    if (!(atomicOr(flag_words + (lo >> 2), bit) & bit)) atomicAdd(marked, 1u);
    if (tile_pos) tile_pos[(int64_t)blockIdx.x * 256 + threadIdx.x] = lo;
  }
}

// Bits of `mask` below this lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// One wave per CSR row: 64 entries at a time, destinations from wave ballots, so each row keeps its
// column order.
__global__ __launch_bounds__(256) void k_place_entries(const PlaceEntries a) {
  const int row = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  if (row >= a.m) return;
  const int b = a.rowptr[row], e = a.rowptr[row + 1];
  const int si = a.split_index[row];
  if (si >= 0) {
    int cur[kXcds];
#pragma unroll
    for (int x = 0; x < kXcds; ++x) cur[x] = a.cursor[si * kXcds + x];
    for (int p = b; p < e; p += 64) {
      const int q = p + lane;
      const bool in = q < e;
      const int32_t c = in ? a.col[q] : 0;
      const int xq = xcd_of_column(c);
      int dst = 0;
#pragma unroll
      for (int x = 0; x < kXcds; ++x) {
        const uint64_t mask = __ballot(in && xq == x);
        if (in && xq == x) dst = cur[x] + lanes_below(mask);
        cur[x] += __popcll(mask);
      }
      if (in) {
        a.col_out[dst] = c;
        if (a.val_out) a.val_out[dst] = half_bits_of(__builtin_bit_cast(uint32_t, a.val[q]));
        if (a.x_pos) a.x_pos[dst - a.x_base] = q;
        if (a.x_src) a.x_src[a.merge_off[si] + (q - b)] = (int32_t)(dst - a.x_base);
      }
    }
    if (a.compact) return;
  }
  int out = a.main_rowptr[row];
  for (int p = b; p < e; p += 64) {
    const int q = p + lane;
    const bool keep = q < e && !(a.flag && a.flag[q]);
    const uint64_t mask = __ballot(keep);
    if (keep) {
      const int dst = out + lanes_below(mask);
      a.col_out[dst] = a.col[q];
      if (a.val_out) a.val_out[dst] = half_bits_of(__builtin_bit_cast(uint32_t, a.val[q]));
      if (a.res_pos) a.res_pos[dst] = q;
    }
    out += __popcll(mask);
  }
}

// Column histogram for the hot-row choice (global atomics: plan creation only).
// Workgroup b counts into copy b % copies of the histogram (copies of n counts each), so that the
// atomics on a hot column spread over that many addresses (R-MAT 2^20's hottest columns take tens
// of thousands of entries each: 4.0 ms with one copy).
__global__ __launch_bounds__(256) void k_count_columns(const int32_t* __restrict__ col, int64_t total, int32_t n,
                                                       int32_t* __restrict__ counts, int copies) {
  int32_t* h = counts + (int64_t)(blockIdx.x % copies) * n;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int32_t c = col[e];
    if (c >= 0 && c < n) atomicAdd(&h[c], 1);
  }
}

// counts[c] = sum of the copies' counts of column c (copy 0 is counts itself).
__global__ __launch_bounds__(256) void k_sum_copies(int32_t* __restrict__ counts, int32_t n, int copies) {
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < n; c += (int64_t)gridDim.x * 256) {
    int32_t s = 0;
    for (int k = 0; k < copies; ++k) s += counts[(int64_t)k * n + c];
    counts[c] = s;
  }
}

// Takes the residual entries of MFMA-window rows back out of a column histogram: the window kernel
// gathers them through the plain column ids, never from the staged rows.  One workgroup per window.
__global__ __launch_bounds__(256) void k_uncount_windows(const MfmaWindow* __restrict__ mwin, int32_t m,
                                                         const int32_t* __restrict__ rowptr,
                                                         const int32_t* __restrict__ col, int32_t n,
                                                         int32_t* __restrict__ counts) {
  const MfmaWindow w = mwin[blockIdx.x];
  const int32_t r1 = min(w.row0 + 16, m);
  if (w.row0 >= r1) return;
  for (int32_t e = rowptr[w.row0] + (int32_t)threadIdx.x; e < rowptr[r1]; e += 256) {
    const int32_t c = col[e];
    if (c >= 0 && c < n) atomicSub(&counts[c], 1);
  }
}

__global__ __launch_bounds__(256) void k_renumber_hot(const int32_t* __restrict__ col, int64_t total, int32_t n,
                                                      const int32_t* __restrict__ rank, int32_t* __restrict__ hot_col) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int32_t c = col[e];
    const int32_t r = c >= 0 && c < n ? rank[c] : -1;
    hot_col[e] = r >= 0 ? ~r : c;
  }
}

__global__ __launch_bounds__(256) void k_check_columns(const int32_t* __restrict__ col, int64_t total, int32_t n,
                                                       unsigned long long* __restrict__ first_bad) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int32_t c = col[e];
    if (c < 0 || c >= n) atomicMin(first_bad, (unsigned long long)e);
  }
}

// One wave per chunk of a candidate row (long rows are cut into chunks, so that a hub row does not
// hold one wave for its whole length).  Columns are flagged with relaxed byte stores of 1 (many
// chunks flag the same hot columns; a store does not wait on the ones before it, as an atomic OR
// to the same words did: 5.5 ms for R-MAT 2^20's 20M candidate entries).
__global__ __launch_bounds__(256) void k_split_stats(const int32_t* __restrict__ col, const int32_t* __restrict__ start,
                                                     const int32_t* __restrict__ len, const int32_t* __restrict__ row,
                                                     int32_t chunks, int32_t* __restrict__ cnt,
                                                     uint8_t* __restrict__ seen) {
  const int32_t i = (int32_t)(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (i >= chunks) return;
  const int l = threadIdx.x & 63;
  const int32_t* c = col + start[i];
  const int32_t n = len[i];
  int32_t k[kXcds] = {};
  for (int32_t q = l; q < n; q += 64) {
    const int32_t v = c[q];
    const int x = xcd_of_column(v);
#pragma unroll
    for (int y = 0; y < kXcds; ++y) k[y] += x == y;
    if (seen) __hip_atomic_store(seen + v, (uint8_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int y = 0; y < kXcds; ++y) {
    int32_t v = k[y];
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
    if (l == 0 && v) atomicAdd(&cnt[(int64_t)row[i] * kXcds + y], v);
  }
}

// *out += nonzero bytes of flags[0, n) (each 0 or 1), read as 32-bit words (n padded to 4 bytes).
__global__ __launch_bounds__(256) void k_count_flags(const uint32_t* __restrict__ words, int64_t nwords,
                                                     unsigned long long* __restrict__ out) {
  unsigned long long s = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nwords; i += (int64_t)gridDim.x * 256)
    s += __popc(words[i] & 0x01010101u);
  for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d);
  if ((threadIdx.x & 63) == 0 && s) atomicAdd(out, s);
}

__global__ __launch_bounds__(256) void k_group_tile_fill(const int32_t* __restrict__ tile_win,
                                                         const int32_t* __restrict__ tile_group,
                                                         const int32_t* __restrict__ s_offsets,
                                                         const int8_t* __restrict__ s_pos, int32_t ntiles,
                                                         float min_fill, uint8_t* __restrict__ pass) {
  const int32_t t = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (t >= ntiles) return;
  const int32_t g0 = tile_group[t];
  const int32_t g1 = min(g0 + 4, s_offsets[tile_win[t] + 1]);
  int kept = 0;
  for (int32_t g = g0; g < g1; ++g) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(s_pos + (int64_t)g * 32);
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = p[i];   // four int8 positions, -1 = none
      kept += ((w & 0x80u) == 0) + ((w & 0x8000u) == 0) + ((w & 0x800000u) == 0) + ((w & 0x80000000u) == 0);
    }
  }
  pass[t] = (float)kept < min_fill * 256.f ? 0 : 1;
}

__global__ __launch_bounds__(256) void k_gather_group_tiles(const int32_t* __restrict__ ids, int32_t nids,
                                                            const int32_t* __restrict__ tile_win,
                                                            const int32_t* __restrict__ tile_group,
                                                            const int32_t* __restrict__ s_offsets,
                                                            const int32_t* __restrict__ s_col,
                                                            const float* __restrict__ s_val,
                                                            const int8_t* __restrict__ s_pos,
                                                            GroupTile* __restrict__ out) {
  const int32_t i = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (i >= nids) return;
  const int32_t t = ids[i];
  const int32_t w = tile_win[t], g0 = tile_group[t];
  const int32_t ng = min(4, s_offsets[w + 1] - g0);
  GroupTile& o = out[i];
  o.row0 = w * 16;
  o.ngroups = ng;
  for (int g = 0; g < 4; ++g) {
    for (int p = 0; p < 4; ++p) o.cols[g * 4 + p] = g < ng ? s_col[(int64_t)(g0 + g) * 4 + p] : -1;
    for (int j = 0; j < 32; ++j) {
      o.val[g][j] = g < ng ? s_val[(int64_t)(g0 + g) * 32 + j] : 0.f;
      o.pos[g][j] = g < ng ? s_pos[(int64_t)(g0 + g) * 32 + j] : (int8_t)-1;
    }
  }
}

__global__ __launch_bounds__(256) void k_zero_fill(float* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) out[i] = 0.f;
}
#endif  // TRS_KERNEL_PART == 0

}  // namespace

// Each load width's launchers -- and so its kernel instantiations -- are compiled in an object of
// their own (this file with TRS_KERNEL_PART = the width), part 0 holds the rest and calls them.
template <int VEC>
hipError_t spmm_width(const DevicePlan& p, const uint16_t* B, int64_t ldb, int K, float* C, int64_t ldc,
                      float* partial, uint16_t* hot, hipStream_t s, hipEvent_t* ev);
template <int VEC>
hipError_t sddmm_width(const DevicePlan& p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy, int K,
                       float* out, uint16_t* hot, float* xbuf, hipStream_t s, hipEvent_t* ev);
#if TRS_KERNEL_PART > 0
template <int VEC>
hipError_t spmm_width(const DevicePlan& p, const uint16_t* B, int64_t ldb, int K, float* C, int64_t ldc,
                      float* partial, uint16_t* hot, hipStream_t s, hipEvent_t* ev) {
  return launch_spmm_vec<VEC>(p, B, ldb, K, C, ldc, partial, hot, s, ev);
}
template <int VEC>
hipError_t sddmm_width(const DevicePlan& p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy, int K,
                       float* out, uint16_t* hot, float* xbuf, hipStream_t s, hipEvent_t* ev) {
  return launch_sddmm_vec<VEC>(p, X, ldx, Y, ldy, K, out, hot, xbuf, s, ev);
}
#endif
#define TRS_WIDTH_INSTANCES(PREFIX, V)                                                                       \
  PREFIX template hipError_t spmm_width<V>(const DevicePlan&, const uint16_t*, int64_t, int, float*, int64_t, \
                                           float*, uint16_t*, hipStream_t, hipEvent_t*);                      \
  PREFIX template hipError_t sddmm_width<V>(const DevicePlan&, const uint16_t*, int64_t, const uint16_t*,     \
                                            int64_t, int, float*, uint16_t*, float*, hipStream_t, hipEvent_t*);
#if TRS_KERNEL_PART > 0
TRS_WIDTH_INSTANCES(, TRS_KERNEL_PART)
#else
TRS_WIDTH_INSTANCES(extern, 8)
TRS_WIDTH_INSTANCES(extern, 4)
TRS_WIDTH_INSTANCES(extern, 2)
TRS_WIDTH_INSTANCES(extern, 1)

hipError_t launch_zero_fill(float* out, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(k_zero_fill, dim3((unsigned)blocks), dim3(256), 0, stream, out, n);
  return hipGetLastError();
}

static unsigned stride_grid(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

hipError_t launch_count_columns(const int32_t* col, int64_t total, int32_t n, int32_t* counts, int copies,
                                hipStream_t stream) {
  if (total <= 0 || n <= 0) return hipSuccess;
  if (copies < 1) copies = 1;
  hipLaunchKernelGGL(k_count_columns, dim3(stride_grid(total)), dim3(256), 0, stream, col, total, n, counts, copies);
  if (copies > 1) hipLaunchKernelGGL(k_sum_copies, dim3(stride_grid(n)), dim3(256), 0, stream, counts, n, copies);
  return hipGetLastError();
}

hipError_t launch_uncount_windows(const MfmaWindow* mwin, int32_t nmwin, int32_t m, const int32_t* rowptr,
                                  const int32_t* col, int32_t n, int32_t* counts, hipStream_t stream) {
  if (nmwin <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_uncount_windows, dim3((unsigned)nmwin), dim3(256), 0, stream, mwin, m, rowptr, col, n, counts);
  return hipGetLastError();
}

hipError_t launch_renumber_hot(const int32_t* col, int64_t total, int32_t n, const int32_t* rank, int32_t* hot_col,
                               hipStream_t stream) {
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_renumber_hot, dim3(stride_grid(total)), dim3(256), 0, stream, col, total, n, rank, hot_col);
  return hipGetLastError();
}

hipError_t launch_check_columns(const int32_t* col, int64_t total, int32_t n, unsigned long long* first_bad,
                                hipStream_t stream) {
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_check_columns, dim3(stride_grid(total)), dim3(256), 0, stream, col, total, n, first_bad);
  return hipGetLastError();
}

hipError_t launch_split_stats(const int32_t* col, const int32_t* start, const int32_t* len, const int32_t* row,
                              int32_t chunks, int32_t* cnt, uint8_t* seen, hipStream_t stream) {
  if (chunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_split_stats, dim3((unsigned)((chunks + 3) / 4)), dim3(256), 0, stream, col, start, len, row,
                     chunks, cnt, seen);
  return hipGetLastError();
}

hipError_t launch_count_flags(const uint8_t* flags, int64_t n, unsigned long long* out, hipStream_t stream) {
  const int64_t nwords = (n + 3) / 4;
  if (nwords <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_count_flags, dim3(stride_grid(nwords)), dim3(256), 0, stream,
                     reinterpret_cast<const uint32_t*>(flags), nwords, out);
  return hipGetLastError();
}

hipError_t launch_group_tile_fill(const int32_t* tile_win, const int32_t* tile_group, const int32_t* s_offsets,
                                  const int8_t* s_pos, int32_t ntiles, float min_fill, uint8_t* pass,
                                  hipStream_t stream) {
  if (ntiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_group_tile_fill, dim3((unsigned)((ntiles + 255) / 256)), dim3(256), 0, stream, tile_win,
                     tile_group, s_offsets, s_pos, ntiles, min_fill, pass);
  return hipGetLastError();
}

hipError_t launch_gather_group_tiles(const int32_t* ids, int32_t nids, const int32_t* tile_win,
                                     const int32_t* tile_group, const int32_t* s_offsets, const int32_t* s_col,
                                     const float* s_val, const int8_t* s_pos, GroupTile* out, hipStream_t stream) {
  if (nids <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_group_tiles, dim3((unsigned)((nids + 255) / 256)), dim3(256), 0, stream, ids, nids,
                     tile_win, tile_group, s_offsets, s_col, s_val, s_pos, out);
  return hipGetLastError();
}

hipError_t launch_mark_tile_entries(const TileEntries* tiles, int32_t ntiles, int32_t m, const int32_t* rowptr,
                                    const int32_t* col, uint32_t* flag_words, uint32_t* marked, int32_t* tile_pos,
                                    hipStream_t stream) {
  if (ntiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_mark_tile_entries, dim3((unsigned)ntiles), dim3(256), 0, stream, tiles, m, rowptr, col,
                     flag_words, marked, tile_pos);
  return hipGetLastError();
}

hipError_t launch_place_entries(const PlaceEntries& a, hipStream_t stream) {
  if (a.m <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_place_entries, dim3((unsigned)((a.m + 3) / 4)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_spmm(const DevicePlan& p, const uint16_t* B, int64_t ldb, int K, float* C, int64_t ldc,
                       float* partial, uint16_t* hot, hipStream_t stream, hipEvent_t* ev) {
  // wide loads only where they leave at least 4 lanes per group (whose column/value loads are
  // shared): with K <= 8 one or two lanes would stream a task alone (R-MAT K=8: 0.545 ms with one
  // 16-byte load per entry, 0.348 with two lanes of 8-byte loads, 0.283 with eight lanes of 2-byte
  // loads, 0.273 with four lanes of 4-byte loads (below); K=4 0.515 -> 0.220), and K=16 runs best
  // as 4 lanes of 8-byte loads (R-MAT 0.436 ms with 2 lanes of 16-byte loads, 0.324; grid+hubs
  // 0.368 -> 0.307)
  const bool v8 = K > 16 && K % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0 && aligned16(B) && aligned16(C) &&
                  (partial == nullptr || aligned16(partial));
  // 8-byte loads when rows are only 8-byte aligned (K % 4 == 0): R-MAT K=100 3.22 ms with 2-byte
  // loads
  const bool v4 = K > 8 && K % 4 == 0 && ldb % 4 == 0 && ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(B) & 7) == 0 &&
                  aligned16(C) && (partial == nullptr || aligned16(partial));
  // 4-byte loads for even widths that 8-byte loads cannot serve (same-box A/B against 2-byte
  // loads, R-MAT: K=10 0.438 -> 0.346 ms, K=18 0.776 -> 0.612, K=30 0.828 -> 0.641, K=98 3.245 ->
  // 2.313; SBM K=18 0.295 -> 0.208).  K=12 and 16 stay on 8-byte loads in 4-lane groups (R-MAT
  // K=16 0.318 vs 0.333 ms with 4-byte loads in 8-lane groups)
  // K = 6 and 8 too, in groups of 4 lanes (R-MAT K=6 0.297 -> 0.253 ms, K=8 0.283 -> 0.273; SBM,
  // whose window kernel stages B rows with the same loads, K=6 0.189 -> 0.144, K=8 0.180 ->
  // 0.145; grid+hubs K=8 0.241 -> 0.245).  K=4 stays on 2-byte loads (R-MAT 0.219 vs 0.233)
  const bool v2 = (K > 8 || K == 6 || K == 8) && !(v8 || v4) && K % 2 == 0 && ldb % 2 == 0 && ldc % 2 == 0 &&
                  (reinterpret_cast<uintptr_t>(B) & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 7) == 0 &&
                  (partial == nullptr || aligned16(partial));
  // (the staged hot rows need 16-byte aligned rows in the buffer too)
  if (hot != nullptr && !aligned16(hot)) hot = nullptr;
  if (v2) return spmm_width<2>(p, B, ldb, K, C, ldc, partial, nullptr, stream, ev);
  return v8 ? spmm_width<8>(p, B, ldb, K, C, ldc, partial, hot, stream, ev)
       : v4 ? spmm_width<4>(p, B, ldb, K, C, ldc, partial, nullptr, stream, ev)
            : spmm_width<1>(p, B, ldb, K, C, ldc, partial, nullptr, stream, ev);
}

hipError_t launch_sddmm(const DevicePlan& p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy,
                        int K, float* out, uint16_t* hot, float* xbuf, hipStream_t stream, hipEvent_t* ev) {
  // K <= 8 takes 2-byte loads so that K lanes share a task (R-MAT K=8: 0.747 ms with one lane of
  // 16-byte loads per task, 0.331), and up to K=64 8-byte loads are faster than 16-byte ones
  // (same-box A/B on R-MAT: K=32 0.468 -> 0.430 ms, K=64 0.550 -> 0.503; K=128 1.038 vs 1.080
  // with 8-byte loads, so 16-byte loads from K=72 on)
  const bool v8 = K > 64 && K % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && aligned16(X) && aligned16(Y);
  const bool v4 = K > 8 && K % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 7) == 0 &&
                  (reinterpret_cast<uintptr_t>(Y) & 7) == 0;
  // 4-byte loads for K = 9..16 (8-lane groups, whose outputs go out in 32-byte runs; R-MAT K=16
  // 0.418 -> 0.334 ms, K=12 0.408 -> 0.287) and for other even widths that 8-byte loads cannot
  // serve (K=18 0.743 -> 0.431 ms, K=66 1.866 -> 1.479, K=130 2.350 -> 1.993 with 2-byte loads)
  const bool v2 = K > 8 && (K <= 16 || !(v8 || v4)) && K % 2 == 0 && ldx % 2 == 0 && ldy % 2 == 0 &&
                  (reinterpret_cast<uintptr_t>(X) & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 3) == 0;
  if (hot != nullptr && !aligned16(hot)) hot = nullptr;
  if (v2) return sddmm_width<2>(p, X, ldx, Y, ldy, K, out, nullptr, xbuf, stream, ev);
  return v8 ? sddmm_width<8>(p, X, ldx, Y, ldy, K, out, hot, xbuf, stream, ev)
       : v4 ? sddmm_width<4>(p, X, ldx, Y, ldy, K, out, nullptr, xbuf, stream, ev)
            : sddmm_width<1>(p, X, ldx, Y, ldy, K, out, nullptr, xbuf, stream, ev);
}
#endif  // TRS_KERNEL_PART == 0

}  // namespace trs
