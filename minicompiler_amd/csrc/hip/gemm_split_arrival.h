// Split-K arrival for the FP32 GEMM bodies: the blocks that compute the K
// ranges of one C tile each store their range's partial sums, then count
// themselves in on the tile's counter; the last to arrive adds the ranges'
// partials in range order (the fixed order of the separate sum launch, so
// the same bits) and stores C through the epilogue. Nothing waits on another
// block: every block arrives once and goes on, and only the last one reads.
// No headers, so hipRTC compiles it as is; the generator puts it before the
// body that uses it.
//
// Visibility across the XCDs (each has its own L2): the partials are stored
// and loaded with device-scope (agent) accesses, which the hardware keeps
// coherent across the L2s (stores write through to memory, loads bypass
// stale lines), and the count goes up only after each wave's stores have
// completed (vmcnt(0)). The last block loads only after its atomic returned
// the final count. A release / acquire fence pair would also order the
// block's other memory traffic, at the price of writing back and
// invalidating a whole L2 per fence: on an MI355X that made a 16x4096x4096
// split launch 3.5x slower than adding the splits in a separate launch.
//
// Counters: one unsigned per tile, zero before the launch; the last block
// of a tile puts its counter back to zero, so consecutive launches (stream
// order, graph replays) find them zero again. Two launches that share
// counters must not overlap.
#pragma once

// A partial sum stored for, and loaded by, the tile's last block.
__device__ __forceinline__ void mc_split_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float mc_split_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of the block, after its partial stores
// (mc_split_store). True, in every thread, in the last of the tile's `depth`
// blocks to arrive; that block may then read every range's partial with
// mc_split_load. `flag`: an LDS int.
__device__ __forceinline__ bool mc_split_last_arrival(unsigned* counter, int depth, int* flag) {
    // This wave's partial stores have completed before the barrier (the
    // signal fences keep the compiler from moving memory accesses across).
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) {
        // A vector atomic from one lane, at device (agent) scope.
        const unsigned before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before + 1u == static_cast<unsigned>(depth);
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last ? 1 : 0;
    }
    __syncthreads();
    return *flag != 0;
}
