// sxq_sync_dev.h -- device helpers for handing data from the workgroups of one launch
// to the last of them to arrive, and for controlling which loads a wait covers.
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
// publish_and_count waits until this thread's stores have completed (vmcnt 0, as an asm
// statement with a memory clobber, so the compiler can neither sink a store below it nor
// hoist a later access above it), joins the workgroup (so every thread's stores have),
// then thread 0 bumps the counter; the last arriver only issues its loads after the
// counter returned.  What this relies on beyond the HIP memory model: agent-scope
// relaxed accesses reach the device-coherent level in program order once their vmcnt
// wait has passed, and the last arriver's loads, which depend on the counter's value
// through control flow and the memory clobbers, are not issued before it returns.
SXQ_DEV void store_agent(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SXQ_DEV void store_agent(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
SXQ_DEV float load_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SXQ_DEV int load_agent(const int* p) { return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Every thread of the workgroup calls it; `flag` is a workgroup-shared bool.  `total` =
// number of workgroups that count on this counter.
SXQ_DEV bool publish_and_count(unsigned* counter, unsigned total, bool* flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores are complete
    __syncthreads();                // ... and so are everyone else's in the workgroup
    if (threadIdx.x == 0)
        *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    return *flag;
}

// 16-byte loads and stores coherent at agent scope (sc1), through a buffer resource over
// `bytes` bytes at `base` (offsets in bytes; out-of-range loads return zeros).  The
// compiler tracks their completion like any other load.
SXQ_DEV __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
SXQ_DEV float4 load16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
    return make_float4(v.x, v.y, v.z, v.w);
}
SXQ_DEV void store16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const f4 w = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, w), r, off, 0, 16);
}

// A 16-byte load through the global address space, whatever the pointer's type: a
// generic pointer (one read from memory rather than passed as a kernel argument) would
// give a flat load, which also counts against the LDS counter, so that every later LDS
// wait would wait for it too.  Loaded as a native vector: HIP's uint4/float4 copy
// through a generic reference, which would drop the address space again.
template <typename T>
SXQ_DEV T ld_global(const T* p) {
    static_assert(sizeof(T) == 16, "16-byte loads");
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u v = *(const __attribute__((address_space(1))) v4u*)(const void*)p;
    return __builtin_bit_cast(T, v);
}

// The loads issued above this point stay issued above it: neither the optimizer (which
// would sink a load to its first use, e.g. behind a prologue's arithmetic on other
// loads) nor the instruction scheduler moves a memory access or an instruction across
// it.  It waits for nothing.
SXQ_DEV void issue_point() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// The same (wave-uniform) pointer with its provenance hidden from the optimizer: loads
// through it are ordinary memory reads, which issue_point keeps on their side, where
// loads through a const __restrict__ kernel argument count as invariant and move freely.
template <typename T>
SXQ_DEV T* opaque_ptr(T* p) {
    asm volatile("" : "+s"(p));
    return p;
}

// Workgroup barrier without __syncthreads()'s memory fence: loads in flight stay in
// flight (the fence would wait for all of them).
SXQ_DEV void barrier_nofence() { asm volatile("s_barrier" ::: "memory"); }

}  // namespace sxq
