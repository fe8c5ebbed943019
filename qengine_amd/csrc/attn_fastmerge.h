// attn_fastmerge.h -- the cross-workgroup merge of the single-launch decode
// fast paths (TQ3 and Q8_0 caches).  Every workgroup of a launch writes one
// record per (q head, query, key chunk) {m, l, o[256]}; the last workgroups of
// the grid are designated mergers, one per (q head, query, 128-dim block)
// unit, and turn the unit's records into the fp16 output.
//
// Records move between workgroups (possibly on different XCDs, whose L2s are
// not coherent with each other) with buffer accesses carrying the sc0|sc1
// cache policy: stores write through to the device coherence point and loads
// read from it.  A writer stores a record's data, waits for those stores to
// complete (s_waitcnt vmcnt(0)) and only then stores the record's two tags
// (one per 128-block unit); a merger loads a record's data only after it has
// read its unit's tag.  Once a merger has seen every tag of its unit it clears
// them (the other unit of the same records has tag words of its own), so that
// after a launch every tag is clear again: the state the next launch, ordered
// after this one on the stream, starts from, and the state of a zero-filled
// workspace.  No counter or epoch is involved, and no workgroup pays an L2
// write-back or invalidate (what agent-scope fences cost on this GPU).
// Only mergers wait, and they are dispatched after every other workgroup, so
// progress does not depend on workgroup co-residency.  Their wait is bounded:
// a merger that runs out of polls writes NaN rows and sets the sticky error
// word of the workspace header (one relaxed agent-scope store), which the host
// reads with qkv_decode_workspace_status and clears with
// qkv_decode_workspace_reset.
#pragma once
#include "attn_common.h"
#include "qkv_device.h"

namespace qkv {

constexpr int kCoherent = 1 | 16;   // sc0 | sc1

// Diagnostic build (-DQKV_PHASE_TRACE): byte offset, inside the merge area,
// where a merger leaves the time its polls completed; the next two words hold
// the time its record rows had arrived and the time the waves' partials were
// folded (before the normalise / rotate / store of the output rows).
constexpr int kTracePolledByte = 16384;

// Record index of (q head, query t, chunk) in the fast-path workspace.
__device__ __forceinline__ long rec_index(const AttnArgs& p, int qh, int t, int chunk) {
  return (long)(qh * p.sub_n + t) * p.n_slots + chunk;
}

// Ragged (paged) launches: the sub_n * n_chunks record shares of a kv head
// are split over the slots in proportion to their key counts (every slot at
// least one, at most 128), so that long slots get more workgroups than short
// ones; every workgroup computes the same split.  Slot s owns the shares
// first .. first+count-1, whose records sit at rec_index(p, qh, 0, share).
__device__ __forceinline__ int slot_keys(const AttnArgs& p, int s) {
  return min(max(p.ctx_lens[s], 0), p.ctx_max);
}
__device__ inline int share_count(const AttnArgs& p, int s, long total) {
  const int extra = p.sub_n * p.n_chunks - p.sub_n;
  return min(128, 1 + (total > 0 ? (int)((long)extra * slot_keys(p, s) / total) : 0));
}
__device__ inline long total_keys(const AttnArgs& p) {
  long total = 0;
  for (int i = 0; i < p.sub_n; i++) total += slot_keys(p, i);
  return total;
}
__device__ inline void slot_shares(const AttnArgs& p, int s, int& first, int& count) {
  const long total = total_keys(p);
  int acc = 0;
  for (int i = 0; i < s; i++) acc += share_count(p, i, total);
  first = acc;
  count = share_count(p, s, total);
}
// The slot of share g (-1 past the last slot's shares), its first share and count.
__device__ inline int share_slot(const AttnArgs& p, int g, int& first, int& count) {
  const long total = total_keys(p);
  int acc = 0;
  for (int i = 0; i < p.sub_n; i++) {
    const int w = share_count(p, i, total);
    if (g < acc + w) {
      first = acc;
      count = w;
      return i;
    }
    acc += w;
  }
  first = count = 0;
  return -1;
}

// Merger thread layout for a THREADS-thread workgroup: slices of 32 threads
// (one dim quad of a 128-block each), 128/slices records per thread
// (n_chunks <= 128).  The reduction area holds one 128-float partial per wave.
template <int THREADS>
struct MergeLayout {
  static constexpr int kSlices = THREADS / 32;
  static constexpr int kRecPerThread = 128 / kSlices;
  static constexpr int kWaves = THREADS / 64;
  static constexpr int kRedFloats = kWaves * 128;
};

// Workgroup-wide AND of `pred` over a 1-D workgroup of THREADS threads: one
// LDS word per wave (`slots`, free while the call runs), no work-item id
// beyond threadIdx.x (the device library's __syncthreads_and forms a linear
// id from all three, which keeps them live across a whole kernel).
template <int THREADS>
__device__ __forceinline__ bool block_and(bool pred, int* slots) {
  const bool wave_all = __builtin_amdgcn_ballot_w64(!pred) == 0;
  __syncthreads();   // the previous use of the slots is over
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = wave_all ? 1 : 0;
  __syncthreads();
  bool all = true;
#pragma unroll
  for (int w = 0; w < THREADS / 64; w++) all = all && slots[w] != 0;
  return all;
}

// NaN rows for unit (query t, q head qh, 128-block blk): threads 0..15 store 8 halves each.
__device__ __forceinline__ void write_nan_unit(const AttnArgs& p, int t, int qh, int blk, uint16_t* out) {
  if (threadIdx.x < 16)
    *reinterpret_cast<uint4*>(out + ((long)t * p.num_q + qh) * 256 + blk * 128 + threadIdx.x * 8) =
        make_uint4(0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u);
}

// Merge the n <= 128 records base .. base+n-1 of one unit (q head qh, query
// t, 128-block blk) and write its fp16 output  o = sum w_c o_c / sum w_c l_c,
// w_c = 2^(m_c - M), rotated back (o = rs*D*H*o per 128-block) when ROTATE.
// 1. Threads 0..n-1 poll one record each ({m, l, tags} in one 16-byte load)
//    until every tag of the unit is set; m and l go to LDS (mls, 128
//    entries); then each clears its record's tag of this unit.
// 2. Thread (record slice sl = tid/32, dim quad dq = tid%32) loads the rows
//    of records sl, sl+slices, ... in one round.  Every wave reduces the
//    record scalars to M and L itself (lane l: records l and l+64), weights
//    its rows, and folds its two slices together (lanes l and l^32); the
//    waves' partials meet once in LDS, where 16 threads sum them, normalise,
//    rotate and store.
// If the records did not all appear within the poll limit: clears the tags it
// did see, writes NaN rows, records the error in the workspace header and
// returns false.
template <int THREADS, bool ROTATE>
__device__ bool merge_unit(float* red, f2_t* mls, const AttnArgs& p, __amdgpu_buffer_rsrc_t rml,
                           __amdgpu_buffer_rsrc_t ro, long base, int n, int qh, int t, int blk,
                           uint16_t* out) {
  using ML = MergeLayout<THREADS>;
  constexpr int kSlices = ML::kSlices, kRecPerThread = ML::kRecPerThread, kWaves = ML::kWaves;
  constexpr int kHD = 256;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int sl = tid >> 5, dq = tid & 31;
  bool seen = tid >= n;
  bool complete = false;
  for (int spins = 0; spins < p.spin_limit; spins++) {
    if (!seen) {
      const f4_t r = __builtin_amdgcn_raw_buffer_load_b128(
          rml, (uint32_t)((base + tid) * kRecMlBytes), 0, kCoherent);
      if (__float_as_uint(blk ? r[3] : r[2]) == kTagValid) {
        seen = true;
        mls[tid] = f2_t{r[0], r[1]};
      }
    }
    // (red is free until the rows are folded: it holds the vote)
    if (block_and<THREADS>(seen, reinterpret_cast<int*>(red))) {
      complete = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
#ifdef QKV_PHASE_TRACE
  if (tid == 0)
    *reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(red) + kTracePolledByte) =
        __builtin_amdgcn_s_memrealtime();
#endif
  if (!complete) {
    if (tid < n && seen)   // the tags this merger saw will not be read again
      __builtin_amdgcn_raw_buffer_store_b32(0u, rml, (uint32_t)((base + tid) * kRecMlBytes + 8 + 4 * blk),
                                            0, kCoherent);
    write_nan_unit(p, t, qh, blk, out);
    if (tid == 0)
      __hip_atomic_store(p.ws_header + kWsErrorWord, kWsErrorTimeout, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();   // mls is reused by the next unit
    return false;
  }
  if (tid < n)   // this unit has seen its records: clear their tags for the next launch
    __builtin_amdgcn_raw_buffer_store_b32(0u, rml, (uint32_t)((base + tid) * kRecMlBytes + 8 + 4 * blk), 0,
                                          kCoherent);
  f4_t v[kRecPerThread];
#pragma unroll
  for (int i = 0; i < kRecPerThread; i++) {
    const int c = sl + kSlices * i;
    v[i] = c < n ? __builtin_amdgcn_raw_buffer_load_b128(
                       ro, (uint32_t)(((base + c) * kHD + blk * 128 + 4 * dq) * 4), 0, kCoherent)
                 : f4_t{0.f, 0.f, 0.f, 0.f};
  }
#ifdef QKV_PHASE_TRACE
  __builtin_amdgcn_s_waitcnt(0);   // (trace build only: the rows' arrival, thread 0's view)
  if (tid == 0)
    *reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(red) + kTracePolledByte + 8) =
        __builtin_amdgcn_s_memrealtime();
#endif
  // common max M and weight sum L over the records (empty chunks, l = 0,
  // carry no weight), in every wave
  const f2_t r0 = lane < n ? mls[lane] : f2_t{-INFINITY, 0.f};
  const f2_t r1 = lane + 64 < n ? mls[lane + 64] : f2_t{-INFINITY, 0.f};
  const bool a0 = r0[1] > 0.f, a1 = r1[1] > 0.f;
  const float M = wave_max(fmaxf(a0 ? r0[0] : -INFINITY, a1 ? r1[0] : -INFINITY));
  const float L = wave_sum((a0 ? __builtin_amdgcn_exp2f(r0[0] - M) * r0[1] : 0.f) +
                           (a1 ? __builtin_amdgcn_exp2f(r1[0] - M) * r1[1] : 0.f));
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kRecPerThread; i++) {
    const int c = sl + kSlices * i;
    if (c < n) {
      const f2_t r = mls[c];
      if (r[1] > 0.f) acc += __builtin_amdgcn_exp2f(r[0] - M) * v[i];
    }
  }
  // the wave's two slices: lanes l and l^32 hold the same dim quad
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e]), __float_as_uint(acc[e]),
                                                     false, false);
    acc[e] = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
  }
  if (lane < 32) *reinterpret_cast<f4_t*>(&red[wave * 128 + 4 * dq]) = acc;
  __syncthreads();
#ifdef QKV_PHASE_TRACE
  if (tid == 0)
    *reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(red) + kTracePolledByte + 16) =
        __builtin_amdgcn_s_memrealtime();
#endif
  // 16 lanes x 8 elements (threads 0..15): sum the waves' partials, normalise,
  // rotate back, store fp16
  if (tid < 16) {
    // TQ3 values (ROTATE) were summed over the kCenScale-scaled centroid table
    const float inv = (L > 0.f ? 1.0f / L : 0.f) * (ROTATE ? kCenScaleInv : 1.0f);
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const f4_t lo = *reinterpret_cast<const f4_t*>(&red[w * 128 + tid * 8]);
      const f4_t hi = *reinterpret_cast<const f4_t*>(&red[w * 128 + tid * 8 + 4]);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[i] += lo[i];
        x[4 + i] += hi[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] *= inv;
    uint32_t pk[4];
    if constexpr (ROTATE) {
      wht8_inreg(x);
      wht_xor_lanes16(x, tid);
      const float rs = wht_scale();
      const uint32_t sbits = sign_word_sel(tid >> 2) >> (8 * (tid & 3));   // signs of elements tid*8..+7
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float y[2];
#pragma unroll
        for (int e2 = 0; e2 < 2; e2++) {
          const bool pos = (sbits >> (2 * i + e2)) & 1u;
          const float vv = x[2 * i + e2] * rs;
          y[e2] = pos ? vv : -vv;
        }
        pk[i] = f2h(y[0]) | (f2h(y[1]) << 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) pk[i] = f2h(x[2 * i]) | (f2h(x[2 * i + 1]) << 16);
    }
    *reinterpret_cast<uint4*>(out + ((long)t * p.num_q + qh) * kHD + blk * 128 + tid * 8) =
        make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
  __syncthreads();   // red and mls are reused by the next unit
  return true;
}

// Store this workgroup's merged rows as records: row r = qi * gqa + hh (q head
// h*gqa + hh of query t0 + qi) with data mo[r][256], maxima Mv[r] (log2
// units) and sums Lv[r]; data first, then (once every thread's data stores
// are complete) the tags of both 128-block units.
template <int THREADS>
__device__ void store_records(const float* mo, const float* Mv, const float* Lv,
                              const AttnArgs& p, __amdgpu_buffer_rsrc_t rml,
                              __amdgpu_buffer_rsrc_t ro, int h, int t0, int rows, int chunk) {
  constexpr int kHD = 256;
  const int gqa = p.num_q / p.num_kv;
  for (int idx = threadIdx.x; idx < rows * 64; idx += THREADS) {
    const int r = idx >> 6, d4 = (idx & 63) * 4;
    const long rec = rec_index(p, h * gqa + r % gqa, t0 + r / gqa, chunk);
    __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const f4_t*>(&mo[r * kHD + d4]), ro,
                                           (uint32_t)((rec * kHD + d4) * 4), 0, kCoherent);
    if (d4 == 0)
      __builtin_amdgcn_raw_buffer_store_b64(f2_t{Mv[r], Lv[r]}, rml,
                                            (uint32_t)(rec * kRecMlBytes), 0, kCoherent);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's data stores are complete
  __syncthreads();
  if ((int)threadIdx.x < rows) {
    const int r = threadIdx.x;
    __builtin_amdgcn_raw_buffer_store_b64(
        u2_t{kTagValid, kTagValid}, rml,
        (uint32_t)(rec_index(p, h * gqa + r % gqa, t0 + r / gqa, chunk) * kRecMlBytes + 8), 0, kCoherent);
  }
}

// One 4-float piece of a record (row of q head qh, query t, chunk), written
// straight from a merge: data at dims d4..d4+3 and, from the thread with
// d4 == 0, the scalars.  publish_records then tags the workgroup's records.
__device__ __forceinline__ void store_record_piece(const AttnArgs& p, __amdgpu_buffer_rsrc_t rml,
                                                   __amdgpu_buffer_rsrc_t ro, int qh, int t, int chunk,
                                                   int d4, f4_t o, float M, float L) {
  const long rec = rec_index(p, qh, t, chunk);
  __builtin_amdgcn_raw_buffer_store_b128(o, ro, (uint32_t)((rec * 256 + d4) * 4), 0, kCoherent);
  if (d4 == 0)
    __builtin_amdgcn_raw_buffer_store_b64(f2_t{M, L}, rml, (uint32_t)(rec * kRecMlBytes), 0, kCoherent);
}

// Tag this workgroup's records (rows 0..rows-1 as in store_records) once every
// thread's data stores are complete; every thread of the workgroup calls it.
// gqa = num_q / num_kv, passed in uniform (scalar register).
__device__ __forceinline__ void publish_records(const AttnArgs& p, __amdgpu_buffer_rsrc_t rml, int h,
                                                int gqa, int t0, int rows, int chunk) {
  __builtin_amdgcn_s_waitcnt(0);  // this thread's data stores are complete
  __syncthreads();
  if ((int)threadIdx.x < rows) {
    const int r = threadIdx.x;
    __builtin_amdgcn_raw_buffer_store_b64(
        u2_t{kTagValid, kTagValid}, rml,
        (uint32_t)(rec_index(p, h * gqa + r % gqa, t0 + r / gqa, chunk) * kRecMlBytes + 8), 0, kCoherent);
  }
}

// The designated mergers: the last min(units, grid) workgroups merge the
// (q head, query, block) units.
template <int THREADS, bool ROTATE>
__device__ void merge_phase(float* red, f2_t* mls, const AttnArgs& p, __amdgpu_buffer_rsrc_t rml,
                            __amdgpu_buffer_rsrc_t ro, uint16_t* out) {
  const int n_units = p.num_q * p.sub_n * 2;
  const int n_mergers = min(n_units, (int)gridDim.x);
  const int mid = (int)blockIdx.x - ((int)gridDim.x - n_mergers);
  if (mid < 0) return;
  // a workspace left inconsistent by an earlier timeout yields NaN rows until it is reset
  const bool poisoned = __hip_atomic_load(p.ws_header + kWsErrorWord, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) != 0;
  // (num_q re-read here: a divisor the compiler would otherwise prepare at
  // kernel entry and hold in a register through the whole tile loop)
  int num_q = p.num_q;
  asm volatile("" : "+s"(num_q));
  for (int u = mid; u < n_units; u += n_mergers) {
    const int blk = u & 1, qh = (u >> 1) % num_q, t = (u >> 1) / num_q;
    long base = rec_index(p, qh, t, 0);
    int n = p.n_chunks;
    if (p.ctx_lens) {   // ragged slots: the slot's shares of the kv head's records
      int first;
      slot_shares(p, t, first, n);
      base = rec_index(p, qh, 0, first);
    }
    if (poisoned)
      write_nan_unit(p, t, qh, blk, out);
    else
      merge_unit<THREADS, ROTATE>(red, mls, p, rml, ro, base, n, qh, t, blk, out);
  }
}

// ---- two units at once --------------------------------------------------
// Mergers with two or more units (a multi-query call: 512 units of the
// 16-token verify over 256 mergers) take them two at a time, one per half of
// the workgroup: each half polls, loads and folds its own unit with reduction
// and scalar areas of its own, and both halves pass the same barriers.
struct MergeUnit {
  long base;
  int n, qh, t, blk;
  bool valid;
};

template <int THREADS, bool ROTATE>
__device__ void merge_unit_pair(float* red_all, f2_t* mls_all, const AttnArgs& p, __amdgpu_buffer_rsrc_t rml,
                                __amdgpu_buffer_rsrc_t ro, const MergeUnit& u0, const MergeUnit& u1,
                                uint16_t* out) {
  constexpr int kTU = THREADS / 2;   // threads per unit (whole waves)
  using ML = MergeLayout<kTU>;
  constexpr int kSlices = ML::kSlices, kRecPerThread = ML::kRecPerThread, kWaves = ML::kWaves;
  constexpr int kHD = 256;
  const bool second = (int)threadIdx.x >= kTU;
  // (selects, not an indexed pair: an indexed array of two units goes to scratch)
  const bool valid = second ? u1.valid : u0.valid;
  const long base = second ? u1.base : u0.base;
  const int n = valid ? (second ? u1.n : u0.n) : 0;
  const int qh = second ? u1.qh : u0.qh, t = second ? u1.t : u0.t, blk = second ? u1.blk : u0.blk;
  float* red = red_all + (second ? ML::kRedFloats : 0);
  f2_t* mls = mls_all + (second ? 128 : 0);
  const int tid = (int)threadIdx.x - (second ? kTU : 0);
  const int lane = tid & 63, wave = tid >> 6;
  const int sl = tid >> 5, dq = tid & 31;
  bool seen = tid >= n;
  bool all0 = false, all1 = false;
  int* slots = reinterpret_cast<int*>(red_all);   // (free until the rows are folded: it holds the vote)
  for (int spins = 0; spins < p.spin_limit; spins++) {
    if (!seen) {
      const f4_t r = __builtin_amdgcn_raw_buffer_load_b128(
          rml, (uint32_t)((base + tid) * kRecMlBytes), 0, kCoherent);
      if (__float_as_uint(blk ? r[3] : r[2]) == kTagValid) {
        seen = true;
        mls[tid] = f2_t{r[0], r[1]};
      }
    }
    const bool wave_all = __builtin_amdgcn_ballot_w64(!seen) == 0;
    __syncthreads();   // the previous use of the slots is over
    if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = wave_all ? 1 : 0;
    __syncthreads();
    all0 = all1 = true;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      all0 = all0 && slots[w] != 0;
      all1 = all1 && slots[kWaves + w] != 0;
    }
    if (all0 && all1) break;
    __builtin_amdgcn_s_sleep(1);
  }
  const bool complete = second ? all1 : all0;
  if (!complete) {
    if (tid < n && seen)   // the tags this merger saw will not be read again
      __builtin_amdgcn_raw_buffer_store_b32(0u, rml, (uint32_t)((base + tid) * kRecMlBytes + 8 + 4 * blk),
                                            0, kCoherent);
    if (valid && tid < 16)
      *reinterpret_cast<uint4*>(out + ((long)t * p.num_q + qh) * 256 + blk * 128 + tid * 8) =
          make_uint4(0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u);
    if (tid == 0)
      __hip_atomic_store(p.ws_header + kWsErrorWord, kWsErrorTimeout, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  } else if (tid < n) {   // this unit has seen its records: clear their tags for the next launch
    __builtin_amdgcn_raw_buffer_store_b32(0u, rml, (uint32_t)((base + tid) * kRecMlBytes + 8 + 4 * blk), 0,
                                          kCoherent);
  }
  const int nr = complete ? n : 0;   // a timed-out half folds nothing (it passes the barrier below)
  f4_t v[kRecPerThread];
#pragma unroll
  for (int i = 0; i < kRecPerThread; i++) {
    const int c = sl + kSlices * i;
    v[i] = c < nr ? __builtin_amdgcn_raw_buffer_load_b128(
                        ro, (uint32_t)(((base + c) * kHD + blk * 128 + 4 * dq) * 4), 0, kCoherent)
                  : f4_t{0.f, 0.f, 0.f, 0.f};
  }
  const f2_t r0 = lane < nr ? mls[lane] : f2_t{-INFINITY, 0.f};
  const f2_t r1 = lane + 64 < nr ? mls[lane + 64] : f2_t{-INFINITY, 0.f};
  const bool a0 = r0[1] > 0.f, a1 = r1[1] > 0.f;
  const float M = wave_max(fmaxf(a0 ? r0[0] : -INFINITY, a1 ? r1[0] : -INFINITY));
  const float L = wave_sum((a0 ? __builtin_amdgcn_exp2f(r0[0] - M) * r0[1] : 0.f) +
                           (a1 ? __builtin_amdgcn_exp2f(r1[0] - M) * r1[1] : 0.f));
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kRecPerThread; i++) {
    const int c = sl + kSlices * i;
    if (c < nr) {
      const f2_t r = mls[c];
      if (r[1] > 0.f) acc += __builtin_amdgcn_exp2f(r[0] - M) * v[i];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e]), __float_as_uint(acc[e]),
                                                     false, false);
    acc[e] = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
  }
  __syncthreads();   // every wave has left the vote: red may take the partials
  if (lane < 32) *reinterpret_cast<f4_t*>(&red[wave * 128 + 4 * dq]) = acc;
  __syncthreads();
  if (complete && tid < 16) {
    const float inv = (L > 0.f ? 1.0f / L : 0.f) * (ROTATE ? kCenScaleInv : 1.0f);
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const f4_t lo = *reinterpret_cast<const f4_t*>(&red[w * 128 + tid * 8]);
      const f4_t hi = *reinterpret_cast<const f4_t*>(&red[w * 128 + tid * 8 + 4]);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[i] += lo[i];
        x[4 + i] += hi[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] *= inv;
    uint32_t pk[4];
    if constexpr (ROTATE) {
      wht8_inreg(x);
      wht_xor_lanes16(x, tid);
      const float rs = wht_scale();
      const uint32_t sbits = sign_word_sel(tid >> 2) >> (8 * (tid & 3));   // signs of elements tid*8..+7
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float y[2];
#pragma unroll
        for (int e2 = 0; e2 < 2; e2++) {
          const bool pos = (sbits >> (2 * i + e2)) & 1u;
          const float vv = x[2 * i + e2] * rs;
          y[e2] = pos ? vv : -vv;
        }
        pk[i] = f2h(y[0]) | (f2h(y[1]) << 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) pk[i] = f2h(x[2 * i]) | (f2h(x[2 * i + 1]) << 16);
    }
    *reinterpret_cast<uint4*>(out + ((long)t * p.num_q + qh) * kHD + blk * 128 + tid * 8) =
        make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
  __syncthreads();   // red and mls are reused by the next units
}

// merge_phase with the units taken two at a time while at least two remain
// for this merger (mergers: 2 * ML<THREADS / 2>::kRedFloats floats at `red`,
// 256 record scalars at `mls`).
template <int THREADS, bool ROTATE>
__device__ void merge_phase_paired(float* red, f2_t* mls, const AttnArgs& p, __amdgpu_buffer_rsrc_t rml,
                                   __amdgpu_buffer_rsrc_t ro, uint16_t* out) {
  static_assert(THREADS % 128 == 0, "two halves of whole waves");
  const int n_units = p.num_q * p.sub_n * 2;
  const int n_mergers = min(n_units, (int)gridDim.x);
  const int mid = (int)blockIdx.x - ((int)gridDim.x - n_mergers);
  if (mid < 0) return;
  const bool poisoned = __hip_atomic_load(p.ws_header + kWsErrorWord, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) != 0;
  int num_q = p.num_q;
  asm volatile("" : "+s"(num_q));
  auto unit = [&](int u) {   // a contiguous (not ragged) launch
    MergeUnit m{};
    m.valid = u < n_units;
    const int uu = m.valid ? u : 0;
    m.blk = uu & 1;
    m.qh = (uu >> 1) % num_q;
    m.t = (uu >> 1) / num_q;
    m.base = rec_index(p, m.qh, m.t, 0);
    m.n = p.n_chunks;
    return m;
  };
  for (int u = mid; u < n_units; u += 2 * n_mergers) {
    const MergeUnit a = unit(u), b = unit(u + n_mergers);
    if (poisoned) {
      write_nan_unit(p, a.t, a.qh, a.blk, out);
      if (b.valid) write_nan_unit(p, b.t, b.qh, b.blk, out);
    } else if (b.valid) {
      merge_unit_pair<THREADS, ROTATE>(red, mls, p, rml, ro, a, b, out);
    } else {
      merge_unit<THREADS, ROTATE>(red, mls, p, rml, ro, a.base, a.n, a.qh, a.t, a.blk, out);
    }
  }
}

}  // namespace qkv
