// Per-workgroup phase stamps of the staged decode, compiled in only with
// -DKVSSD_TIMELINE (csrc/build.py --timeline writes that build to
// kvssd/libkvssd_hip_timeline.so; csrc/timeline.py runs a workload with it and
// prints the phases).  KVSSD_STAMP(slot) stores the 100 MHz real-time clock
// when wave 0 of the workgroup passes the slot; without the flag it is empty.
#pragma once

#include <cstdint>

namespace kvssd {

constexpr int kTimelineWgs = 4096;
constexpr int kTimelineSlots = 64;

// slots of a decoding workgroup
constexpr int kStampEntry = 0;
constexpr int kStampLoop = 1;        // prologue done, entering the stage loop
constexpr int kStampStage = 2;       // + k: stage k's barrier passed (k < 16; later stages share slot 17)
constexpr int kStampLoopEnd = 18;    // last stage computed
constexpr int kStampStored = 19;     // partial stores issued
constexpr int kStampStage0Issued = 22;  // prologue: stage 0 copies issued
constexpr int kStampRowsLanded = 23;    // query rows and valid counts landed
constexpr int kStampStage1Issued = 24;  // query operands built, stage 1 issued
constexpr int kStampStage0Landed = 25;  // stage 0 landed (before the loop)

}  // namespace kvssd

#ifdef KVSSD_TIMELINE
extern __device__ uint64_t kvssd_timeline_stamps[kvssd::kTimelineWgs * kvssd::kTimelineSlots];
#define KVSSD_STAMP(slot)                                                                                \
  do {                                                                                                   \
    if (threadIdx.x == 0 && blockIdx.x < static_cast<unsigned>(kvssd::kTimelineWgs))                     \
      kvssd_timeline_stamps[blockIdx.x * kvssd::kTimelineSlots + (slot)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define KVSSD_STAMP(slot) \
  do {                    \
  } while (0)
#endif
