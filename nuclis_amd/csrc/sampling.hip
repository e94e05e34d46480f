// Device sampling helpers beside the greedy argmax: the history penalties
// and the partial top-k with its softmax denominator.
//
// penalize: Sampler.penalize (inference/src/sampling/root.zig:375-381) on
// every logit whose id is in the history bit set (bit id of word id / 32),
// in place, one thread per logit, in F32 with IEEE division.
//
// top-k: the k best logits by (value descending, index ascending), the order
// of the CPU sampler (sampling/root.zig:385-387). Each logit becomes a
// 64-bit key whose unsigned order is that order: the high word is the
// complement of the float's order-preserving bit pattern (-0 folded onto +0,
// since the sampler compares floats, and NaN mapped past every value so it
// never enters the list), the low word the index. Workgroups sort chunks of
// 4096 keys in LDS with a bitonic network and keep their first k; the
// passes repeat over the surviving keys until one chunk is left, whose
// first k are the answer. The exp-sum pass then writes the 64 F32 partial
// sums of exp((l - max) / T) and non-finite flags that the host adds in F64
// (sampling/root.zig:154-173).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace nuq {

namespace {

constexpr uint32_t TOPK_CHUNK = 4096, TOPK_THREADS = 1024;
constexpr uint64_t TOPK_PAD = ~0ull;

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t i) {
    uint32_t hi;
    if (v != v) {
        hi = 0xffffffffu;  // NaN: after every value
    } else {
        uint32_t u = __float_as_uint(v);
        if (v == 0.0f) u = 0;  // -0 ties with +0
        const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        hi = ~ord;  // larger values first
    }
    return ((uint64_t)hi << 32) | i;
}

// Sorts s[0, width) ascending (width a power of two, <= TOPK_CHUNK) with
// the workgroup's TOPK_THREADS threads. Thread t of a stage compares keys i
// and i + stride, i = t with a zero inserted at the stride's bit. While
// stride <= 64 the keys a wave touches are the same two blocks of 128 in
// every stage, so those stages need only the wave's own LDS ordering; a
// stage that spans waves (or is followed by one) takes a workgroup barrier.
__device__ __forceinline__ void bitonic_sort(uint64_t *s, uint32_t width, uint32_t tid) {
    __syncthreads();
    for (uint32_t size = 2; size <= width; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = tid; t < width / 2; t += TOPK_THREADS) {
                const uint32_t i = ((t & ~(stride - 1)) << 1) | (t & (stride - 1)), j = i + stride;
                const uint64_t a = s[i], b = s[j];
                const bool ascending = (i & size) == 0;
                if ((a > b) == ascending) {
                    s[i] = b;
                    s[j] = a;
                }
            }
            if (stride > 64 || (stride == 1 && size < width && size > 64)) {
                __syncthreads();
            } else {
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    __syncthreads();
}

__global__ void __launch_bounds__(256) penalize_kernel(float *__restrict__ logits, uint32_t count,
                                                       const uint32_t *__restrict__ history, float repetition,
                                                       float presence) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    if (!(history[i >> 5] & (1u << (i & 31u)))) return;
    const float x = logits[i];
    const float scaled = x > 0.0f ? x / repetition : x * repetition;
    logits[i] = scaled - presence;
}

// One chunk of up to TOPK_CHUNK keys per workgroup: from the logits (first
// pass, `logits` non-null) or from the previous pass's keys. The first k of
// the sorted chunk go to keys_out, or, in the final pass, to values/indices
// (the value read back from the logits, so -0 stays -0; NaN and padding
// entries become (-inf, 0xffffffff)).
//
// state (when non-null) is {candidate count, done}: the candidate pass reads
// its n from state[0] and does nothing when it exceeds one chunk; otherwise
// it writes the answer and sets done, and the full passes, launched behind
// it, return at once.
__global__ void __launch_bounds__(TOPK_THREADS) topk_sort_kernel(const float *__restrict__ logits,
                                                                 const uint64_t *__restrict__ keys_in, uint32_t n,
                                                                 uint32_t k, uint64_t *__restrict__ keys_out,
                                                                 const float *__restrict__ source,
                                                                 float *__restrict__ values,
                                                                 uint32_t *__restrict__ indices,
                                                                 uint32_t *__restrict__ state, bool candidates) {
    __shared__ uint64_t s[TOPK_CHUNK];
    const uint32_t tid = threadIdx.x;
    uint32_t width = TOPK_CHUNK;  // keys sorted: the chunk, or the candidates' power of two
    if (state) {
        if (candidates) {
            n = state[0];
            if (n > TOPK_CHUNK) return;  // too many candidates: the full passes run
            width = 256;
            while (width < n) width <<= 1;
        } else if (state[1]) {
            return;  // the candidate pass already answered
        }
    }
    const uint64_t base = (uint64_t)blockIdx.x * TOPK_CHUNK;
    for (uint32_t e = tid; e < width; e += TOPK_THREADS) {
        const uint64_t g = base + e;
        uint64_t key = TOPK_PAD;
        if (g < n) key = logits ? topk_key(logits[g], (uint32_t)g) : keys_in[g];
        s[e] = key;
    }
    bitonic_sort(s, width, tid);
    for (uint32_t r = tid; r < k; r += TOPK_THREADS) {
        const uint64_t key = s[r];
        if (keys_out) {
            keys_out[(uint64_t)blockIdx.x * k + r] = key;
        } else {
            const bool real = (uint32_t)(key >> 32) != 0xffffffffu;
            const uint32_t idx = (uint32_t)key;
            values[r] = real ? source[idx] : -__builtin_inff();
            indices[r] = real ? idx : 0xffffffffu;
        }
    }
    if (state && candidates && tid == 0) state[1] = 1;
}

// The filter's bound: TOPK_GROUPS (>= k) contiguous groups, one wave each,
// reduced to their best keys; the k-th best of those, T, has k distinct
// logits at or above it, so every one of the k best keys is <= T.
constexpr uint32_t TOPK_GROUPS = 1024;
__global__ void __launch_bounds__(64) topk_group_kernel(const float *__restrict__ logits, uint32_t count,
                                                        uint64_t *__restrict__ group_best) {
    const uint32_t g = blockIdx.x, lane = threadIdx.x;
    const uint32_t begin = (uint32_t)((uint64_t)count * g / TOPK_GROUPS);
    const uint32_t end = (uint32_t)((uint64_t)count * (g + 1) / TOPK_GROUPS);
    uint64_t b = TOPK_PAD;
    for (uint32_t i = begin + lane; i < end; i += 64) b = min(b, topk_key(logits[i], i));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) b = min(b, (uint64_t)__shfl_xor((unsigned long long)b, off, 64));
    if (lane == 0) group_best[g] = b;
}

// The bound from the group bests by a two-level radix select: a histogram
// of their top key bytes finds the byte b1 whose bin holds the k-th best, a
// histogram of the next byte within that bin finds b2, and the bound is the
// last key with prefix (b1, b2). At least k group bests (distinct logits)
// lie at or below it, so the k best keys all do. Stores it in state words
// 2-3 and resets the candidate count and the done flag (words 0-1).
__global__ void __launch_bounds__(TOPK_GROUPS) topk_select_kernel(const uint64_t *__restrict__ group_best, uint32_t k,
                                                                  uint32_t *__restrict__ state) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t pick[2];  // chosen byte, rank still needed within it
    __shared__ uint32_t wave_total[4], scan_h[256], scan_inc[256];
    const uint32_t tid = threadIdx.x;
    const uint64_t key = group_best[tid];
    uint32_t need = k;
    uint32_t prefix = 0;
#pragma unroll
    for (int level = 0; level < 2; ++level) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        const bool in = level == 0 || (uint32_t)(key >> 56) == prefix;
        const uint32_t bin = (uint32_t)(key >> (56 - 8 * level)) & 255u;
        // one LDS atomic per distinct bin per wave (the bests cluster in few bins)
        uint64_t pending = __ballot(in);
        while (pending) {
            const uint32_t leader = (uint32_t)__builtin_ctzll(pending);
            const uint32_t b = (uint32_t)__shfl((int)bin, (int)leader, 64);
            const uint64_t same = __ballot(in && bin == b) & pending;
            if ((threadIdx.x & 63) == leader) atomicAdd(&hist[b], (uint32_t)__builtin_popcountll(same));
            pending &= ~same;
        }
        __syncthreads();
        // inclusive scan of the 256 bins (4 waves), then the bin where it
        // reaches `need` records itself
        if (tid < 256) {
            const uint32_t lane = tid & 63, h = hist[tid];
            uint32_t inc = h;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t v = (uint32_t)__shfl_up((int)inc, off, 64);
                if (lane >= (uint32_t)off) inc += v;
            }
            if (lane == 63) wave_total[tid >> 6] = inc;
            scan_h[tid] = h;
            scan_inc[tid] = inc;
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t before = 0;
            for (uint32_t w = 0; w < (tid >> 6); ++w) before += wave_total[w];
            const uint32_t inc = scan_inc[tid] + before, exc = inc - scan_h[tid];
            if (exc < need && inc >= need) {
                pick[0] = tid;
                pick[1] = need - exc;
            }
        }
        __syncthreads();
        if (level == 0) prefix = pick[0];
        else prefix = (prefix << 8) | pick[0];
        need = pick[1];
        __syncthreads();
    }
    if (tid == 0) {
        const uint64_t bound = ((uint64_t)prefix << 48) | 0x0000ffffffffffffull;
        state[0] = 0;
        state[1] = 0;
        state[2] = (uint32_t)bound;
        state[3] = (uint32_t)(bound >> 32);
    }
}

// Keys <= the bound go to the candidate list (at most TOPK_CHUNK are kept;
// the count keeps counting so an overflow is seen). One wave per
// workgroup takes TOPK_FILTER_SPAN logits, 16 per lane, and reserves its
// candidates with one atomic.
constexpr uint32_t TOPK_FILTER_PER = 16, TOPK_FILTER_SPAN = 64 * TOPK_FILTER_PER;
__global__ void __launch_bounds__(64) topk_filter_kernel(const float *__restrict__ logits, uint32_t count,
                                                         uint64_t *__restrict__ cand, uint32_t *__restrict__ state) {
    const uint32_t lane = threadIdx.x;
    const uint64_t bound = ((uint64_t)state[3] << 32) | state[2];
    const uint32_t first = blockIdx.x * TOPK_FILTER_SPAN + lane;
    uint64_t keys[TOPK_FILTER_PER];
    uint64_t masks[TOPK_FILTER_PER];
    uint32_t total = 0;
#pragma unroll
    for (uint32_t j = 0; j < TOPK_FILTER_PER; ++j) {
        const uint32_t i = first + 64 * j;
        keys[j] = i < count ? topk_key(logits[i], i) : TOPK_PAD;
        masks[j] = __ballot(i < count && keys[j] <= bound);
        total += (uint32_t)__builtin_popcountll(masks[j]);
    }
    if (total == 0) return;
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&state[0], total);
    base = __shfl(base, 0, 64);
#pragma unroll
    for (uint32_t j = 0; j < TOPK_FILTER_PER; ++j) {
        if ((masks[j] >> lane) & 1) {
            const uint32_t pos = base + (uint32_t)__builtin_popcountll(masks[j] & ((1ull << lane) - 1));
            if (pos < TOPK_CHUNK) cand[pos] = keys[j];
        }
        base += (uint32_t)__builtin_popcountll(masks[j]);
    }
}

// Partition p of `partials` sums exp((x - max) / T) over logits p*256 + tid,
// stepping by partials*256, and flags a non-finite logit. The partition
// shape and the F32 operation order are the reference's
// (kernels/sampling.metal:144-170); the host adds the partials in F64.
__global__ void __launch_bounds__(256) expsum_kernel(const float *__restrict__ logits, uint32_t count,
                                                     const float *__restrict__ top_values, float temperature,
                                                     uint32_t partials, float *__restrict__ sums,
                                                     uint32_t *__restrict__ flags) {
    __shared__ float part[4];
    __shared__ uint32_t bad[4];
    const uint32_t tid = threadIdx.x;
    const float maximum = top_values[0];
    float sum = 0.0f;
    uint32_t nonfinite = 0;
    for (uint32_t i = blockIdx.x * 256 + tid; i < count; i += partials * 256) {
        const float x = logits[i];
        if (!__builtin_isfinite(x)) nonfinite = 1;
        sum += expf((x - maximum) / temperature);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        sum += __shfl_xor(sum, off, 64);
        nonfinite |= __shfl_xor(nonfinite, off, 64);
    }
    if ((tid & 63) == 0) {
        part[tid >> 6] = sum;
        bad[tid >> 6] = nonfinite;
    }
    __syncthreads();
    if (tid == 0) {
        sums[blockIdx.x] = ((part[0] + part[1]) + part[2]) + part[3];
        flags[blockIdx.x] = bad[0] | bad[1] | bad[2] | bad[3];
    }
}

}  // namespace

hipError_t launch_penalize(hipStream_t s, float *logits, uint32_t count, const uint32_t *history, float repetition,
                           float presence) {
    hipLaunchKernelGGL(penalize_kernel, dim3((count + 255) / 256), dim3(256), 0, s, logits, count, history, repetition,
                       presence);
    return hipGetLastError();
}

// Scratch (u64 units): two key buffers for the full passes, the candidate
// list, the group bounds, and the {count, done} state words.
uint64_t topk_scratch_keys() {
    return 2ull * ((TOPK_MAX_COUNT + TOPK_CHUNK - 1) / TOPK_CHUNK) * TOPK_CAPACITY + TOPK_CHUNK + TOPK_GROUPS + 2;
}

hipError_t launch_topk(hipStream_t s, const float *logits, uint32_t count, uint32_t k, float temperature,
                       uint64_t *scratch, float *values, uint32_t *indices, float *sums, uint32_t *flags) {
    if (count == 0 || count > TOPK_MAX_COUNT || k == 0 || k > TOPK_CAPACITY || k > count) return hipErrorInvalidValue;
    const uint64_t half = ((TOPK_MAX_COUNT + TOPK_CHUNK - 1) / TOPK_CHUNK) * TOPK_CAPACITY;
    uint64_t *bufs[2] = {scratch, scratch + half};
    uint64_t *cand = scratch + 2 * half, *group_best = cand + TOPK_CHUNK;
    uint32_t *state = (uint32_t *)(group_best + TOPK_GROUPS);  // count, done, bound (2 words)
    hipError_t e;
    // Candidate path: group bests, their k-th (the bound), filter, one sorted chunk.
    hipLaunchKernelGGL(topk_group_kernel, dim3(TOPK_GROUPS), dim3(64), 0, s, logits, count, group_best);
    hipLaunchKernelGGL(topk_select_kernel, dim3(1), dim3(TOPK_GROUPS), 0, s, group_best, k, state);
    hipLaunchKernelGGL(topk_filter_kernel, dim3((count + TOPK_FILTER_SPAN - 1) / TOPK_FILTER_SPAN), dim3(64), 0, s,
                       logits, count, cand, state);
    hipLaunchKernelGGL(topk_sort_kernel, dim3(1), dim3(TOPK_THREADS), 0, s, nullptr, cand, 0u, k, nullptr, logits,
                       values, indices, state, true);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // Full passes (they return at once when the candidate path answered).
    uint32_t n = count, chunks = (count + TOPK_CHUNK - 1) / TOPK_CHUNK;
    const uint64_t *in = nullptr;
    int which = 0;
    bool first = true;
    while (true) {
        const bool last = chunks == 1;
        hipLaunchKernelGGL(topk_sort_kernel, dim3(chunks), dim3(TOPK_THREADS), 0, s, first ? logits : nullptr, in, n, k,
                           last ? nullptr : bufs[which], logits, values, indices, state, false);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (last) break;
        in = bufs[which];
        which ^= 1;
        n = chunks * k;
        chunks = (n + TOPK_CHUNK - 1) / TOPK_CHUNK;
        first = false;
    }
    hipLaunchKernelGGL(expsum_kernel, dim3(TOPK_PARTIALS), dim3(256), 0, s, logits, count, values, temperature,
                       TOPK_PARTIALS, sums, flags);
    return hipGetLastError();
}

}  // namespace nuq
