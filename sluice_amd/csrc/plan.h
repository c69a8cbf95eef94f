// The expert product's plan (internal to libsluice_hip): the T*k routed
// (token, expert) pairs grouped by slot into blocks of <= SLUICE_BLOCK_M
// pairs, resident slots ascending, then slots whose rows may still be
// streaming, pairs ascending inside a slot (deterministic).  Built by the
// align kernel of the expert product, or by a router-split gap kernel for
// the ids and map it leaves behind (one launch fewer per layer); both run
// plan_build in one workgroup of kPlanThreads threads.
//
// Layout (int32): [n_blocks, P, n_resident, 0 | P block records {slot
// field, count, pair[16]} | P validity flags (1 = the pair's expert is
// resident)]; the first n_resident blocks are those of slots not pending.
// A slot field carries kPendingBit when the slot's rows may still be
// streaming in.
// The shared experts' blocks are not in the plan: the kernels derive them.
#pragma once

#include "common.h"

namespace sluice_plan {

constexpr int kPlanThreads = 256;
constexpr int kPlanWaves = kPlanThreads / SLUICE_WAVE;
constexpr int kBM = SLUICE_BLOCK_M;
constexpr int kBlockInts = 2 + kBM;
constexpr int kHeader = 4;
constexpr int kPendingBit = 1 << 30;
constexpr int kSlotMask = kPendingBit - 1;

__host__ __device__ inline size_t plan_ints(int P) {
  return (size_t)kHeader + (size_t)kBlockInts * P + (size_t)P;
}

struct Scratch {
  int slot_of[SLUICE_MAX_EXPERTS];  // the map, staged (or the identity)
  int cnt[SLUICE_MAX_SLOTS];
  int boff[SLUICE_MAX_SLOTS];
  int run[SLUICE_MAX_SLOTS];
  int pend[SLUICE_MAX_SLOTS];       // the slot's rows may still be streaming
  int wsum[2][kPlanWaves];
};

// Rank of this lane among the lower lanes of its wave that hold the same
// key (keys < 0 take no part), the number of lanes holding it, and whether
// this lane is the lowest of them.  Wave-uniform loop, one pass per
// distinct key.
__device__ inline int wave_rank(int key, int& count, bool& lowest) {
  const int lane = threadIdx.x & (SLUICE_WAVE - 1);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (SLUICE_WAVE - lane));
  int rank = 0;
  count = 0;
  lowest = false;
  uint64_t todo = __ballot(key >= 0);
  while (todo != 0) {
    const int l = __builtin_ctzll(todo);
    const int k = __shfl(key, l, SLUICE_WAVE);
    const uint64_t m = __ballot(key == k);
    if (key == k) {
      rank = __popcll(m & below);
      count = __popcll(m);
      lowest = lane == l;
    }
    todo &= ~m;
  }
  return rank;
}

// Stages the map (global -> slot, -1 = not resident; nullptr = identity)
// and the pending marks (nonzero = the slot's rows may still be streaming;
// nullptr = none) in the scratch.
__device__ inline void plan_stage(const int32_t* __restrict__ map, int E, int S,
                                  const int32_t* __restrict__ pending, Scratch& sc) {
  for (int e = threadIdx.x; e < E; e += kPlanThreads) sc.slot_of[e] = map != nullptr ? map[e] : e;
  for (int s = threadIdx.x; s < S; s += kPlanThreads)
    sc.pend[s] = pending != nullptr && pending[s] != 0;
}

// Builds the plan of the P pairs `ids` into `plan` over the map and pending
// marks staged in sc.slot_of / sc.pend (written by this workgroup before
// the call; the first barrier below publishes them).  id0 = ids[tid] for
// tid < P (-1 otherwise), as the caller loaded it.  Blocks of pending slots
// come after every other block (so the work on resident experts is
// dispatched first) and carry kPendingBit.  Called by all kPlanThreads
// threads of the workgroup; returns the block count to every thread.
__device__ inline int plan_build_staged(int id0, const int32_t* __restrict__ ids, int P, int E,
                                        int S, Scratch& sc, int32_t* __restrict__ plan) {
  const int tid = threadIdx.x;
  const int lane = tid & (SLUICE_WAVE - 1), wave = tid / SLUICE_WAVE;
  int32_t* blocks = plan + kHeader;
  int32_t* valid = blocks + (size_t)kBlockInts * P;
  for (int s = tid; s < S; s += kPlanThreads) {
    sc.cnt[s] = 0;
    sc.run[s] = 0;
  }
  __syncthreads();
  auto slot_of = [&](int g) {
    if ((unsigned)g >= (unsigned)E) return -1;
    const int s = sc.slot_of[g];
    return (unsigned)s < (unsigned)S ? s : -1;
  };
  for (int p = tid; p < P; p += kPlanThreads) {
    const int s = slot_of(p == tid ? id0 : ids[p]);
    if (s >= 0) atomicAdd(&sc.cnt[s], 1);
  }
  __syncthreads();
  // Exclusive scans of blocks-per-slot, resident slots first, then pending
  // ones; thread t owns slots [t*per, t*per+per).
  const int per = (S + kPlanThreads - 1) / kPlanThreads;
  int mine[2] = {0, 0};
  for (int i = 0; i < per; ++i) {
    const int s = tid * per + i;
    if (s < S) mine[sc.pend[s]] += (sc.cnt[s] + kBM - 1) / kBM;
  }
  int incl[2] = {mine[0], mine[1]};
#pragma unroll
  for (int off = 1; off < SLUICE_WAVE; off <<= 1) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int v = __shfl_up(incl[c], off, SLUICE_WAVE);
      if (lane >= off) incl[c] += v;
    }
  }
  if (lane == SLUICE_WAVE - 1) {
    sc.wsum[0][wave] = incl[0];
    sc.wsum[1][wave] = incl[1];
  }
  __syncthreads();
  int wbase[2] = {0, 0}, tot[2] = {0, 0};
  for (int w = 0; w < kPlanWaves; ++w)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if (w < wave) wbase[c] += sc.wsum[c][w];
      tot[c] += sc.wsum[c][w];
    }
  int acc[2] = {wbase[0] + incl[0] - mine[0], tot[0] + wbase[1] + incl[1] - mine[1]};
  for (int i = 0; i < per; ++i) {
    const int s = tid * per + i;
    if (s < S) {
      const int c = sc.pend[s];
      sc.boff[s] = acc[c];
      acc[c] += (sc.cnt[s] + kBM - 1) / kBM;
    }
  }
  __syncthreads();
  // Ranks in pair order, one chunk of kPlanThreads pairs at a time: within a
  // wave by ballot, across the chunk's waves in wave order (each wave adds
  // its per-slot counts to run[] before the next one reads it).
  for (int c = 0; c < P; c += kPlanThreads) {
    const int p = c + tid;
    const int s = p < P ? slot_of(c == 0 ? id0 : ids[p]) : -1;
    int n_same;
    bool lowest;
    const int wr = wave_rank(s, n_same, lowest);
    const int waves = min(kPlanWaves, (P - c + SLUICE_WAVE - 1) / SLUICE_WAVE);
    for (int w = 0; w < waves; ++w) {
      if (wave == w && s >= 0) {
        const int r = sc.run[s] + wr;
        const int b = sc.boff[s] + r / kBM;
        const int pos = r % kBM;
        int32_t* blk = blocks + (size_t)b * kBlockInts;
        blk[2 + pos] = p;
        if (pos == 0) {
          blk[0] = s | (sc.pend[s] ? kPendingBit : 0);
          const int left = sc.cnt[s] - (r / kBM) * kBM;
          blk[1] = left < kBM ? left : kBM;
        }
        __builtin_amdgcn_wave_barrier();
        if (lowest) sc.run[s] += n_same;
      }
      __syncthreads();
    }
    if (p < P) valid[p] = s >= 0 ? 1 : 0;
  }
  const int nb = tot[0] + tot[1];
  if (tid == 0) {
    plan[0] = nb;
    plan[1] = P;
    plan[2] = tot[0];
    plan[3] = 0;
  }
  return nb;
}

// plan_build_staged over a map and pending marks in global memory.
__device__ inline int plan_build(const int32_t* __restrict__ ids, int P,
                                 const int32_t* __restrict__ map, int E, int S,
                                 const int32_t* __restrict__ pending, Scratch& sc,
                                 int32_t* __restrict__ plan) {
  const int id0 = (int)threadIdx.x < P ? ids[threadIdx.x] : -1;
  plan_stage(map, E, S, pending, sc);
  return plan_build_staged(id0, ids, P, E, S, sc, plan);
}

}  // namespace sluice_plan
