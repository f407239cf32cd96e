// flow.cpp -- the host side of GEMV flows (flow.hip): checks a flow's
// vectors and stages, lays out the device descriptors, tiles each Q4_K stage
// over the CUs, and launches the persistent kernel.
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "flow.hpp"
#include "rt_hip.h"
#include "rt_launch.hpp"

struct rt_hip_flow {
    int device = -1;
    int workgroups = 0;
    int nstages = 0;
    rt_hip::flow::StageD* stages = nullptr;
    rt_hip::flow::SyncD* sync = nullptr;
    uint64_t* arena = nullptr;
};

namespace rt_hip {
namespace {

int fail(int code, const std::string& msg) { return set_error(code, "rt_hip_flow_create: " + msg); }
int hip_fail(hipError_t e, const std::string& what) {
    return set_error(RT_HIP_E_HIP, what + ": " + hipGetErrorString(e));
}

void release(rt_hip_flow* f) {
    if (!f) return;
    hipFree(f->stages);
    hipFree(f->sync);
    hipFree(f->arena);
    delete f;
}

// Weight bytes per workgroup a stage is sized for.
constexpr int64_t kStageBytesPerWg = 16 * 1024;

// Waves per Q4_K tile: enough that the stage's tiles cover every wave of
// the grid, at most one super-block range per wave, every range non-empty.
int pick_ks(int64_t tiles, int nb, int waves, int most) {
    int64_t want = (waves + tiles - 1) / tiles;
    if (want > most) want = most;
    if (want > nb) want = nb;
    if (want < 1) want = 1;
    const int bpw = (nb + static_cast<int>(want) - 1) / static_cast<int>(want);
    return (nb + bpw - 1) / bpw;
}

}  // namespace
}  // namespace rt_hip

extern "C" {

int rt_hip_flow_create(const rt_hip_flow_vector* vectors, int32_t nvectors, const rt_hip_flow_stage* stages,
                       int32_t nstages, rt_hip_flow** out) {
    using namespace rt_hip;
    if (!out) return fail(RT_HIP_E_ARG, "null output handle");
    *out = nullptr;
    if (!vectors || nvectors < 1 || !stages || nstages < 1) return fail(RT_HIP_E_ARG, "need vectors and stages");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_flow_create");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_flow_create");
    const int G = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;

    // internal vectors get arena slots (256-byte aligned each)
    std::vector<int64_t> slot0(nvectors, -1);
    int64_t arena_slots = 0;
    for (int i = 0; i < nvectors; ++i) {
        const int64_t len = vectors[i].len;
        if (len < 1 || len > (int64_t{1} << 24)) return fail(RT_HIP_E_ARG, "vector " + std::to_string(i) + " length");
        if (!vectors[i].external) {
            slot0[i] = arena_slots;
            arena_slots += (len + 31) / 32 * 32;
        }
    }
    rt_hip_flow* f = new rt_hip_flow;
    f->device = dev;
    f->workgroups = G;
    f->nstages = nstages;
    auto alloc = [&](void** p, size_t bytes) {
        e = hipMalloc(p, bytes);
        if (e == hipSuccess) e = hipMemset(*p, 0, bytes);
        return e == hipSuccess;
    };
    if (!alloc(reinterpret_cast<void**>(&f->stages), sizeof(flow::StageD) * nstages) ||
        !alloc(reinterpret_cast<void**>(&f->sync), sizeof(flow::SyncD)) ||
        !alloc(reinterpret_cast<void**>(&f->arena), sizeof(uint64_t) * static_cast<size_t>(arena_slots ? arena_slots : 1))) {
        release(f);
        return e == hipErrorOutOfMemory ? set_error(RT_HIP_E_OOM, "rt_hip_flow_create: device allocation failed")
                                        : hip_fail(e, "rt_hip_flow_create");
    }
    auto slots = [&](int v) -> uint64_t* { return f->arena + slot0[v]; };
    auto reject = [&](int code, const std::string& msg) {
        release(f);
        return fail(code, msg);
    };

    std::vector<int> producer(nvectors, -1);  // stage that writes it
    auto internal = [&](int v) { return v >= 0 && v < nvectors && !vectors[v].external; };
    auto ready = [&](int v, int s) {
        return v >= 0 && v < nvectors && (vectors[v].external || (producer[v] >= 0 && producer[v] < s));
    };
    auto misaligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; };

    std::vector<flow::StageD> sd(nstages);
    for (int s = 0; s < nstages; ++s) {
        const rt_hip_flow_stage& S = stages[s];
        const std::string at = "stage " + std::to_string(s) + ": ";
        flow::StageD& D = sd[s];
        D = flow::StageD{};
        if (S.njobs < 1 || S.njobs > flow::kMaxJobs) return reject(RT_HIP_E_ARG, at + "njobs must be 1..4");
        const int32_t fmt = S.jobs[0].format;
        if (fmt != RT_HIP_Q4K && fmt != RT_HIP_BF16)
            return reject(RT_HIP_E_UNSUPPORTED, at + "format must be Q4K or BF16");
        if (fmt == RT_HIP_BF16 && S.njobs != 1) return reject(RT_HIP_E_ARG, at + "a BF16 stage has one job");
        if (S.k < 1 || S.k > flow::kMaxK) return reject(RT_HIP_E_SHAPE, at + "k must be in [1, 8192]");
        if (fmt == RT_HIP_Q4K && S.k % 256 != 0) return reject(RT_HIP_E_ALIGN, at + "Q4_K k must be a multiple of 256");
        if (fmt == RT_HIP_BF16 && S.k % 8 != 0) return reject(RT_HIP_E_ALIGN, at + "BF16 k must be a multiple of 8");
        if (S.xop < RT_HIP_XOP_NONE || S.xop > RT_HIP_XOP_RMSNORM1)
            return reject(RT_HIP_E_ARG, at + "xop must be NONE, RMSNORM or RMSNORM1");
        if (!ready(S.in0, s) || vectors[S.in0].len != S.k)
            return reject(RT_HIP_E_ARG, at + "in0 must be an external vector or an earlier stage's output of length k");
        if (S.xop != RT_HIP_XOP_NONE && !S.gamma) return reject(RT_HIP_E_ARG, at + "RMSNorm needs gamma");
        if ((S.xop != RT_HIP_XOP_NONE && misaligned(S.gamma)) || misaligned(vectors[S.in0].external))
            return reject(RT_HIP_E_ALIGN, at + "gamma and external inputs must be 16-byte aligned");
        const bool paired = S.act != -1;
        if (paired) {
            if (fmt != RT_HIP_Q4K || S.njobs != 2 || S.jobs[0].n != S.jobs[1].n)
                return reject(RT_HIP_E_ARG, at + "act needs two Q4_K jobs (gate, up) of equal n");
            if (!internal(S.act) || vectors[S.act].len != S.jobs[0].n || producer[S.act] >= 0 ||
                S.act == S.jobs[0].out || S.act == S.jobs[1].out || S.act == S.in0)
                return reject(RT_HIP_E_ARG, at + "act must be a fresh internal vector of length n");
            if (S.jobs[0].add != -1 || S.jobs[1].add != -1)
                return reject(RT_HIP_E_ARG, at + "a paired stage adds no residual");
        }
        D.k = static_cast<int32_t>(S.k);
        D.xop = S.xop;
        D.in_s = vectors[S.in0].external ? nullptr : slots(S.in0);
        D.in_e = vectors[S.in0].external;
        D.act = paired ? slots(S.act) : nullptr;
        D.gamma = S.xop != RT_HIP_XOP_NONE ? S.gamma : nullptr;
        D.eps = S.eps;
        D.kind = fmt == RT_HIP_Q4K ? flow::kQ4K : flow::kBF16;
        D.njobs = S.njobs;
        int64_t units = 0;
        for (int j = 0; j < S.njobs; ++j) {
            const rt_hip_flow_job& J = S.jobs[j];
            const std::string aj = at + "job " + std::to_string(j) + ": ";
            if (J.format != fmt) return reject(RT_HIP_E_ARG, aj + "the jobs of a stage share one format");
            if (!J.w) return reject(RT_HIP_E_ARG, aj + "null weight");
            if (J.n < 1) return reject(RT_HIP_E_ARG, aj + "n must be >= 1");
            if (!internal(J.out) || vectors[J.out].len != J.n)
                return reject(RT_HIP_E_ARG, aj + "out must be an internal vector of length n");
            if (producer[J.out] >= 0) return reject(RT_HIP_E_ARG, aj + "out is written by an earlier job");
            if (J.out == S.in0) return reject(RT_HIP_E_ARG, aj + "out is the input of its own stage");
            for (int q = 0; q < j; ++q)
                if (J.out == S.jobs[q].out) return reject(RT_HIP_E_ARG, aj + "two jobs write one vector");
            if (J.add != -1 && (!ready(J.add, s) || vectors[J.add].len != J.n))
                return reject(RT_HIP_E_ARG, aj + "add must be -1 or an earlier vector of length n");
            flow::JobD& JD = D.job[j];
            JD.w = static_cast<const uint8_t*>(J.w);
            JD.out = slots(J.out);
            if (J.add != -1) {
                JD.add_s = vectors[J.add].external ? nullptr : slots(J.add);
                JD.add_e = vectors[J.add].external;
            }
            JD.plain = J.plain;
            JD.n = static_cast<int32_t>(J.n);
            JD.unit0 = static_cast<int32_t>(units);
            units += fmt == RT_HIP_Q4K ? (J.n + 15) / 16 : J.n;
        }
        for (int j = 0; j < S.njobs; ++j) producer[S.jobs[j].out] = s;
        if (paired) producer[S.act] = s;
        for (int j = S.njobs; j < flow::kMaxJobs; ++j) {
            D.job[j] = D.job[S.njobs - 1];
            D.job[j].unit0 = static_cast<int32_t>(units);  // never reached
        }
        D.units = static_cast<int32_t>(units);
        // Workgroups: about kStageBytesPerWg of weights each (a multiple of 8,
        // one per XCD in turn), at most one per CU.
        int64_t wbytes = 0;
        for (int j = 0; j < S.njobs; ++j)
            wbytes += fmt == RT_HIP_Q4K ? (S.jobs[j].n + 15) / 16 * 16 * (S.k / 256) * 144 : S.jobs[j].n * S.k * 2;
        int64_t wgs = (wbytes + kStageBytesPerWg - 1) / kStageBytesPerWg;
        wgs = (wgs + 7) / 8 * 8;
        if (wgs > G) wgs = G;
        if (wgs < 1) wgs = 1;
        if (fmt == RT_HIP_Q4K) {
            const int nb = static_cast<int>(S.k / 256);
            // paired: tiles of a pair share a round, so at most four waves per tile
            D.ks = pick_ks(units, nb, static_cast<int>(wgs) * flow::kWaves, paired ? 4 : flow::kWaves);
            const int per = (flow::kWaves / D.ks) / (paired ? 2 : 1);
            const int64_t groups = paired ? units / 2 : units;
            if (wgs > groups) wgs = groups;
            int64_t span = wgs * per;
            while ((groups + span - 1) / span > flow::kMaxRounds && wgs < G) {
                wgs = wgs + 8 > G ? G : wgs + 8;
                span = wgs * per;
            }
            if ((groups + span - 1) / span > flow::kMaxRounds)
                return reject(RT_HIP_E_SHAPE, at + "too many Q4_K rows for one stage");
        } else {
            D.ks = 1;
            if (wgs * flow::kWaves > units) wgs = (units + flow::kWaves - 1) / flow::kWaves;
            while (units > static_cast<int64_t>(flow::kMaxRowsPerWave) * wgs * flow::kWaves && wgs < G)
                wgs = wgs + 8 > G ? G : wgs + 8;
            if (units > static_cast<int64_t>(flow::kMaxRowsPerWave) * wgs * flow::kWaves)
                return reject(RT_HIP_E_SHAPE, at + "too many BF16 rows for one stage");
        }
        D.wgs = static_cast<int32_t>(wgs);
    }

    e = hipMemcpy(f->stages, sd.data(), sizeof(flow::StageD) * nstages, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        release(f);
        return hip_fail(e, "rt_hip_flow_create");
    }
    *out = f;
    return RT_HIP_OK;
}

int rt_hip_flow_run(rt_hip_flow* flow, rt_hip_stream stream) {
    using namespace rt_hip;
    if (!flow) return set_error(RT_HIP_E_ARG, "rt_hip_flow_run: null flow");
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_flow_run");
    if (dev != flow->device) return set_error(RT_HIP_E_ARG, "rt_hip_flow_run: the flow belongs to another device");
    e = flow::launch(flow->stages, flow->nstages, flow->sync, flow->workgroups, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? RT_HIP_OK : hip_fail(e, "rt_hip_flow_run");
}

int rt_hip_flow_status(rt_hip_flow* flow) {
    using namespace rt_hip;
    if (!flow) return set_error(RT_HIP_E_ARG, "rt_hip_flow_status: null flow");
    hipError_t e = hipDeviceSynchronize();
    uint32_t err = 0;
    if (e == hipSuccess) e = hipMemcpy(&err, &flow->sync->err, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_flow_status");
    if (err == 0) return RT_HIP_OK;
    const uint32_t zero = 0;
    e = hipMemcpy(&flow->sync->err, &zero, 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "rt_hip_flow_status");
    return set_error(RT_HIP_E_HIP, "rt_hip_flow_status: a wait in stage " + std::to_string(err - 1) +
                                       " ran out (were all workgroups resident?); that run's outputs are undefined");
}

int rt_hip_flow_destroy(rt_hip_flow* flow) {
    rt_hip::release(flow);
    return RT_HIP_OK;
}

}  // extern "C"
