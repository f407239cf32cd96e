// flow.hpp -- device-side descriptors of a GEMV flow (flow.hip): a chain of
// dependent decode GEMV stages run as one persistent launch.  Shared by the
// kernel and the host builder (flow.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rt_hip {
namespace flow {

constexpr int kWaves = 8;             // waves per workgroup; one workgroup per CU
constexpr int kThreads = kWaves * 64;
constexpr int kMaxK = 8192;           // longest input vector
constexpr int kMaxRounds = 8;         // Q4_K tile rounds per stage per workgroup
constexpr int kMaxJobs = 4;
constexpr int kMaxRowsPerWave = 64;   // BF16 rows per wave per stage
enum Kind : int32_t { kQ4K = 0, kBF16 = 1 };

// Descriptors hold direct pointers (no table lookups on the device): a
// vector is either tagged slots in the flow's arena (f32 bits | run tag <<
// 32, written once per run) or plain external f32 memory, ready at launch.
struct JobD {
    const uint8_t* w;       // tiled Q4_K (16-row tiles of K/256 blocks) or row-major bf16
    uint64_t* out;          // output slots
    const uint64_t* add_s;  // residual added to the output: slots, or
    const float* add_e;     //   external values, or neither
    float* plain;           // optional plain f32 copy of the output
    int32_t n;              // output rows
    int32_t unit0;          // the job's first unit in the stage's numbering
};

struct StageD {
    JobD job[kMaxJobs];
    const uint64_t* in_s;   // input: slots, or
    const float* in_e;      //   external values
    uint64_t* act;          // paired gate/up stage: silu(job 0) * job 1 into these slots; else null
    const float* gamma;     // RMSNorm weight (kXRmsNorm / kXRmsNorm1)
    float eps;
    int32_t k, xop, kind, njobs, units, ks;  // units: Q4_K tiles or BF16 rows; ks: waves per tile
    int32_t wgs;            // workgroups that take part in the stage (the first wgs)
};

// Run state, one 128-byte line per word: the run counter (tags are
// epoch + 1), the arrival count of the run's workgroups, and the error word
// (1 + the stage whose wait ran out; 0 when every wait completed).
struct SyncD {
    uint32_t epoch, pad0[31];
    uint32_t arrive, pad1[31];
    uint32_t err, pad2[31];
};

size_t lds_bytes();
hipError_t launch(const StageD* stages, int nstages, SyncD* sync, int workgroups, hipStream_t stream);

}  // namespace flow
}  // namespace rt_hip
