// sxq_sync_dev.h -- device helpers for handing data from the workgroups of one launch
// to the last of them to arrive.
#pragma once
#include "sxq_common.h"

namespace sxq {

// Hand-off between the workgroups of one launch ("the last to arrive finishes the
// job") without a device-wide fence: on this GPU an agent-scope fence writes back or
// invalidates the whole L2 of an XCD, which costs far more than the work it guards.
// Instead the data crosses through accesses that are themselves coherent at agent
// scope -- relaxed agent-scope atomic stores and loads, which go to the coherent level
// rather than a possibly stale L2 -- and the protocol is:
//   writers:  store_agent(data...); publish_and_count() -> true in the last arriver
//   last:     load_agent(data...)
// publish_and_count waits until this thread's stores have completed (s_waitcnt 0),
// joins the workgroup (so every thread's stores have), then thread 0 bumps the counter;
// the last arriver only issues its loads after the counter returned.
SXQ_DEV void store_agent(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SXQ_DEV void store_agent(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SXQ_DEV float load_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SXQ_DEV int load_agent(const int* p) { return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Every thread of the workgroup calls it; `flag` is a workgroup-shared bool.  `total` =
// number of workgroups that count on this counter.
SXQ_DEV bool publish_and_count(unsigned* counter, unsigned total, bool* flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are complete
    __syncthreads();                // ... and so are everyone else's in the workgroup
    if (threadIdx.x == 0)
        *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    return *flag;
}

}  // namespace sxq
