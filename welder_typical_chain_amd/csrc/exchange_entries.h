// exchange_entries.h -- the row exchange of the exchange path
// (chain_tile_kernel's exchange epilogue, fused_matmul_softmax.hip): tagged
// entries, generation words and bounded waits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wtc {

// ---- row exchange ------------------------------------------------------------
// The tiles of a row block (all co-resident) exchange per-row log-sum-exps
// through tagged entries instead of a barrier.  Tile (row block rbg, column
// tile nt) owns slot rbg * nT + nt: 128 64-bit entries, one per tile row, at
// ent + slot * 128.  An entry holds the row's log-sum-exp over the tile's
// columns (f32, log2 domain) in its low word and a tag in its high word, and
// is written with ONE 64-bit atomic store, so a reader sees either an old
// entry or the whole new one.  The tag is the slot's generation + 1: every
// slot has a generation word gen[slot]; the tiles of a row block read the
// generation words of all its slots at kernel start, and the owner of a slot
// increments its word at the end, after reading every other slot of its row
// block.  An entry left by an earlier launch carries a tag <= the slot's
// generation (a slot's entries are only ever written by the tile that owns
// that slot index, whatever the problem shape), so a reader takes an entry
// exactly when its tag equals generation + 1.  No counter, no ordering
// between different words and no cache maintenance is needed, and there is
// no per-launch host state (graph replays work).
//
// Why every reader has read gen[s] before the owner of s increments it: a
// reader's generation loads have returned (the K loop ends with vmcnt(0))
// before it stores its own entries; the owner of s increments gen[s] only
// after loading those entries with this launch's tag.
//
// Readers poll whole half-slots: one wave load takes 64 consecutive rows of
// one slot (512 contiguous bytes), and a half-slot is done when every lane's
// entry carries the expected tag; otherwise the wave sleeps briefly and
// reloads only the half-slots not yet done.  Polling with wide, contiguous
// loads keeps the traffic of the waits small, and there is no round trip
// between learning that the data is there and loading it (the counter
// barrier this replaces needed four: statistics stores acknowledged, counter
// update, generation store, statistics loads).
//
// Every wait is bounded by spin_ticks of the 100 MHz clock; a wait that runs
// out sets bit 0 of err[0], counts in err[2], sets the caller's host-visible
// mailbox word (if any), and the tile goes on with what it has, so the kernel
// always drains.
__device__ inline void store_entry(uint64_t* p, float lse, uint32_t tag) {
  const uint64_t u = (uint64_t)__builtin_bit_cast(uint32_t, lse) | ((uint64_t)tag << 32);
  __hip_atomic_store(p, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t load_entry(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t entry_tag(uint64_t u) { return (uint32_t)(u >> 32); }
__device__ inline float entry_lse(uint64_t u) { return __builtin_bit_cast(float, (uint32_t)u); }

__device__ inline void report_timeout(uint32_t* err, uint32_t* mailbox) {
  __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_add(err + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (mailbox) __hip_atomic_fetch_or(mailbox, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ inline void record_wait(uint32_t* err, uint64_t ticks) {
  const uint32_t w32 = ticks > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)ticks;
  __hip_atomic_fetch_max(err + 1, w32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace wtc
