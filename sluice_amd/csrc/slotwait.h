// Slots whose expert rows are still streaming in (internal to libsluice_hip).
//
// When a router-split gap misses, the host answers the gap kernel as soon as
// the slot bookkeeping is done -- before the rows have landed -- and marks
// each filled slot ready (the gap's stamp in ready[slot], host-mapped
// memory) once the copies of its group of experts completed.  The gap kernel records the
// filled slots in pending[slot] (device memory, the gap's stamp).  The expert
// product then computes the hit experts while the misses stream: its work
// items on a pending slot wait until ready[slot] == pending[slot] and take a
// system-scope acquire before they read the slot's weights.  Only one
// workgroup per slot and gap polls the host-mapped mark (device reads of host
// memory compete with the host-to-device copies for the link); it publishes
// what it saw in device memory, where the other workgroups look.  A gap kernel
// clears the previous gap's pending marks: the product of that gap's step
// waited for every slot it filled.
#pragma once

#include <stdint.h>

struct SlotWait {
  const int32_t* pending = nullptr;     // device [S]; nullptr = no slot streams
  const int32_t* ready = nullptr;       // host-mapped [S]
  int32_t* claim = nullptr;             // device [S]: the stamp a workgroup polls the host for
  int32_t* seen = nullptr;              // device [S]: the stamp whose ready mark was seen
  const int32_t* abort_flag = nullptr;  // host-mapped process-wide abort flag
  int32_t* status = nullptr;            // host-mapped: first failed wait
  // device word: bound of one wait in wall-clock ticks, read by the kernel
  // when it starts to wait, so a graph captured earlier follows the bound
  // set since (sluice_gap_set_timeout rewrites the word)
  const long long* bound = nullptr;
};

// Bound of a wait when a call has no bound word: 20 s at the 100 MHz clock.
constexpr long long kDefaultWaitTicks = 2000000000LL;

// Registry from a layer's device expert map to its slot-wait view (kept by
// the gap layers, read by the expert product).
void slotwait_register(const int32_t* expert_map, const SlotWait& w);
void slotwait_unregister(const int32_t* expert_map);
SlotWait slotwait_lookup(const int32_t* expert_map);
