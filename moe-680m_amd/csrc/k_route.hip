// k_route.hip -- router softmax + top-8 and the prefix-sum expert bucket fill.
#include "moe_internal.hpp"
#include "bucket_fill.hpp"

namespace moe {

// ---------------------------------------------------------------- router top-8
// One 64-lane wave per token.  Replaces shaders/router_topk.comp, whose 256-lane workgroup
// ran two 8-step LDS tree reductions and a serial insertion sort on lane 0
// (router_topk.comp:37-85).  Here each lane keeps E/64 logits in registers; each of the 8
// rounds is a wave max of the order-preserving key (DPP inside rows of 16, then four
// v_readlane) followed by a wave min of the index among lanes holding that key, so the
// lower index wins ties exactly like the shader's strict '>' insertion
// (router_topk.comp:76).  The softmax sum is one DPP + readlane reduction.
template <int NV>
__global__ __launch_bounds__(64) void k_router_topk(const float *__restrict__ logits, int M, int E,
                                                    int renorm, uint16_t *__restrict__ ids,
                                                    float *__restrict__ w) {
    // one wave per workgroup: the dispatcher spreads the tokens over every CU and SIMD
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x;
    if (t >= M) return; // whole wave leaves together
    int sel[TOPK];
    float ws[TOPK];
    route_wave<NV>(logits + (size_t)t * E, E, renorm, lane, sel, ws);
    if (lane < TOPK) {
        float wv = ws[0];
        int id = sel[0];
#pragma unroll
        for (int r = 1; r < TOPK; ++r)
            if (lane == r) { wv = ws[r]; id = sel[r]; }
        ids[(size_t)t * SLOTS + lane] = (uint16_t)id;
        w[(size_t)t * SLOTS + lane] = wv;
    } else if (lane == TOPK) {
        ids[(size_t)t * SLOTS + TOPK] = (uint16_t)E;
        w[(size_t)t * SLOTS + TOPK] = 1.0f;
    }
}

hipError_t launch_router_topk(const float *logits, int M, int E, int renorm, uint16_t *ids, float *w,
                              hipStream_t st, KernelTimer *T) {
    if (M <= 0) return hipSuccess;
    dim3 grid((unsigned)M);
    {
        TimedLaunch tl(T, MOE_K_ROUTER_TOPK, st);
        if (E <= 256)
            hipLaunchKernelGGL(k_router_topk<4>, grid, dim3(64), 0, st, logits, M, E, renorm, ids, w);
        else
            hipLaunchKernelGGL(k_router_topk<16>, grid, dim3(64), 0, st, logits, M, E, renorm, ids, w);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- bucket fill
__global__ __launch_bounds__(BF_THREADS) void k_bucket_fill(BucketArgs a) { bucket_fill_one_wg(a); }
__global__ __launch_bounds__(BF_CHUNK_THREADS) void k_bucket_count(BucketArgs a) { bucket_count_chunk(a, blockIdx.x); }
__global__ __launch_bounds__(BF_THREADS) void k_bucket_scan(BucketArgs a) { bucket_scan_wg(a); }
__global__ __launch_bounds__(BF_CHUNK_THREADS) void k_bucket_scatter(BucketArgs a) { bucket_scatter_chunk(a, blockIdx.x); }

hipError_t launch_bucket_fill(const BucketArgs &a, hipStream_t st, KernelTimer *T) {
    if (a.M < 0) return hipSuccess; // M == 0 still writes all-zero ranges
    TimedLaunch tl(T, MOE_K_BUCKET_FILL, st);
    if (bucket_one_wg(a.M, a.E1)) {
        hipLaunchKernelGGL(k_bucket_fill, dim3(1), dim3(BF_THREADS), bucket_smem(a.E1, true), st, a);
    } else {
        const dim3 grid((unsigned)((a.M + 63) / 64));
        const size_t smem = bucket_chunk_smem(a.E1);
        hipLaunchKernelGGL(k_bucket_count, grid, dim3(BF_CHUNK_THREADS), smem, st, a);
        hipLaunchKernelGGL(k_bucket_scan, dim3(1), dim3(BF_THREADS), bucket_smem(a.E1, false), st, a);
        hipLaunchKernelGGL(k_bucket_scatter, grid, dim3(BF_CHUNK_THREADS), smem, st, a);
    }
    return hipGetLastError();
}

} // namespace moe
