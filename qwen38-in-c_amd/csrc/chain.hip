// chain.hip -- a sequence of decode GEMVs (m <= 8 tokens) in one persistent
// launch: the caller's chain of projections (qwen35-c/src/q35_model.c:877-947
// calls them one after another, each reading what the previous wrote) runs
// without a kernel boundary between them, and the weights of later steps
// stream while earlier steps finish.
//
// Why.  A decode step's projections are dependent launches: each waits for
// the whole previous launch to drain, then pays the command processor's
// dispatch and the first loads' latency, about 2 us per launch beside
// 6-30 us of streaming.  And a launch of 160-192 row-split workgroups (the
// model's qkv, o_proj and down) keeps only those CUs streaming, each with
// two or three blocks per wavefront in flight: latency-bound at ~25 GB/s
// per CU.  The next GEMV's weights do not depend on its activations, so
// nothing but the launch boundary keeps them from streaming early.
//
// Work.  Step s is one row-split GEMV over 1..4 weights sharing x (the
// reference's multi4); its items are the row-split kernel's 32-row
// sub-tiles.  One workgroup per CU (its LDS request leaves room for no
// other), each with a fixed list of items: step s's items are dealt round
// robin over the workgroups, continuing where step s-1's ended, and a
// workgroup's list is in step order.  Four wavefronts stream: each streams
// its K range of every item of the list through one continuous ring of
// DEPTH blocks of weights, block scales and activations in registers.  The
// ring runs across item and step boundaries, so when a workgroup reaches an
// item whose step reads outputs of steps not yet complete, the item's first
// blocks of weights are already loaded; their activations are loaded only
// once the inputs are known complete (until then the ring reads a zero
// buffer in their place, and the blocks already in the ring are reloaded
// after the wait).  Only the arithmetic waits.  A fifth wavefront does the
// rest: it waits for earlier steps (the others wait at a barrier), and
// after each item it adds the four partials, stores the outputs, waits for
// its own stores and counts the item -- a wait for stores would otherwise
// drain a streaming wavefront's ring.
//
// Arithmetic.  Per item exactly the row-split kernel's (gemv_rows.hip):
// the same staging (gemv_rows_common.h), MFMA sequence per block, fmaf per
// block scale and ordered sum of the four wavefronts' partials -- so each
// output has the bits of the same weight's separate row-split call.
//
// Ordering across workgroups (the protocol of the stream-K GEMV's split
// groups).  Outputs are written with agent-scope atomic stores, which go
// through to the device-wide coherence point rather than staying dirty in
// the writer's XCD L2; the fifth wavefront waits for them (s_waitcnt 0)
// before counting the item with an agent-scope atomic add.  The count that
// completes a step sets the step's ready flags (kChainFlags copies on
// separate cache lines: hundreds of workgroups polling one word load its
// memory channel and slow every weight stream that crosses it).  A
// workgroup that needs a step's outputs polls its copy of the flag with
// agent-scope loads, and only then are the activations loaded: with plain
// cached loads where no cache of the device can hold a stale line of them
// (no earlier step of the launch read them, at most one wrote them, and the
// launch's start invalidated the caches), else with agent-scope loads at
// the coherence point.  Barriers here are bare s_barrier (no fence: the
// rings' loads in flight are not waited for).  The last workgroup to finish
// returns the counters and flags to zero, so a launch needs no clearing
// before the next (graph replays included).  A wait gives up after a
// bounded number of polls, setting a host-visible error word (a safety
// net: every item waited on is held by a running workgroup).
#include <algorithm>
#include <type_traits>

#include "gemv_rows_common.h"
#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

using namespace rows;

namespace {

constexpr uint32_t kChainWaves = 4;   // streaming wavefronts; one more does the epilogue

// K blocks per streaming wavefront in flight: as many as its registers hold
// (the fifth wavefront shares a SIMD with one of them, so each has 256).
constexpr uint32_t chain_depth(uint32_t mt) { return mt <= 4 ? 4 : 3; }

// The step table and the item lists are read through the constant address
// space (scalar loads, kept in the scalar cache), and the pointers they hold
// are cast to the global address space: loaded from memory, they would
// otherwise be generic pointers, and every access through them a flat
// instruction.
typedef const __attribute__((address_space(4))) ChainStep *StepPtr;
typedef const __attribute__((address_space(4))) uint32_t *ConstU32;
template <typename T>
__device__ __forceinline__ T *global_ptr(T *p) {
    return (T *)(__attribute__((address_space(1))) T *)p;
}

__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t *ctr(uint8_t *base, uint32_t i) {
    return reinterpret_cast<uint32_t *>(base + (size_t)i * kChainCtrStride);
}

// One K block's activations for all m tokens: element loads (the values of
// load_xblock's element path), cached or at the coherence point.  The same
// number of loads either way, so the compiler's waits stay static.
template <uint32_t MT, bool COHERENT>
__device__ __forceinline__ void load_x(XBlock<MT> &xb, const float *x, uint32_t ldx, uint32_t m, uint32_t k,
                                       uint32_t kb, uint32_t lane) {
    constexpr uint32_t G = XBlock<MT>::kG;
    const uint32_t t = min(lane / XBlock<MT>::kLanesPerToken, m - 1);
    const float *row = x + (size_t)t * ldx;
#pragma unroll
    for (uint32_t e = 0; e < G; e++) {
        const float *a = row + min(kb * kBlock + xcol<MT>(lane, e), k - 1);
        if constexpr (COHERENT)
            xb.v[e] = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            xb.v[e] = *a;
    }
}

// f(integral_constant<I>) for I = B .. E-1, unrolled at compile time.
template <uint32_t B, uint32_t E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<uint32_t, B>());
        static_for<B + 1, E>(f);
    }
}

// The fields of item `it` (step << 16 | sub-tile) of a workgroup's list.
struct ItemRef {
    uint32_t step, si, r0, r1;
};
__device__ __forceinline__ ItemRef item_ref(StepPtr steps, uint32_t e) {
    ItemRef r;
    r.step = e >> 16;
    const uint32_t j = e & 0xFFFFu;
    const StepPtr stp = steps + r.step;
    r.si = 0;
#pragma unroll
    for (uint32_t i = 1; i < 4; i++)
        if (i < stp->nseg && j >= stp->seg[i].cta_begin) r.si = i;
    r.r0 = (j - stp->seg[r.si].cta_begin) * kSubRows;
    r.r1 = min(r.r0 + kSubRows, stp->seg[r.si].rows);
    return r;
}

}  // namespace

// COH: every step's activations and residuals are read at the coherence
// point (some step's may be stale in a cache, see ChainStep::x_mode); else
// all with cached loads.  One kind of load for the whole launch keeps the
// ring's loads one unconditional sequence, whose waits the compiler can
// count exactly (a branch between two kinds of load made it wait for
// nearly every load in flight before each block).
template <uint32_t MT, bool COH>
__global__ __launch_bounds__(64 * (kChainWaves + 1)) void gemv_chain_kernel(ChainParams p) {
    constexpr uint32_t NW = kChainWaves, DEPTH = chain_depth(MT);
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[2][NW][kGemvMaxM][kSubRows];

    const StepPtr steps = (StepPtr)p.steps;
    const uint32_t M = p.m, R = stage_rows(M);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t mrow = lane & 31, hh = lane >> 5;

    const uint32_t i0 = ((ConstU32)p.wg_off)[blockIdx.x];
    const uint32_t nitems = ((ConstU32)p.wg_off)[blockIdx.x + 1] - i0;
    const ConstU32 ilist = (ConstU32)p.wg_items + i0;
    uint32_t ready = 0;   // every step below `ready` is known to have completed

    // Waiting for the outputs of steps [ready, step): the fifth wavefront
    // polls its copy of each step's ready flag, then every wavefront passes
    // the barrier.
    auto wait_steps = [&](uint32_t step) {
        if (wv == NW) {
            for (uint32_t t = ready; t < step; t++) {
                const uint32_t *flag = ctr(p.ready, t * kChainFlags + blockIdx.x % kChainFlags);
                uint32_t spins = 0;
                while (__builtin_amdgcn_readfirstlane((int)ld_agent(flag)) == 0) {
                    __builtin_amdgcn_s_sleep(4);
                    if (++spins > p.spin_limit) {
                        __hip_atomic_store(p.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
        }
        __builtin_amdgcn_s_barrier();
        ready = step;
        // no load below is moved above the polls by the compiler
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    };

    if (wv == NW) {
        // ---- the fifth wavefront: waits, sums, stores, counts ----
        for (uint32_t ci = 0; ci < nitems; ci++) {
            const ItemRef it = item_ref(steps, ilist[ci]);
            const StepPtr stp = steps + it.step;
            if (stp->wait && ready < it.step) wait_steps(it.step);
            __builtin_amdgcn_s_barrier();   // the item's partials are in red[ci & 1]
            float *const y = global_ptr(stp->seg[it.si].y);
            const float *const resid = stp->seg[it.si].resid ? global_ptr(stp->seg[it.si].resid) : nullptr;
            const uint32_t ldy = stp->seg[it.si].ldy;
            constexpr bool coh = COH;
            for (uint32_t o2 = lane; o2 < kSubRows * M; o2 += 64) {
                const uint32_t t = o2 >> 5, nn = o2 & 31;
                float sum = red[ci & 1][0][t][nn];
#pragma unroll
                for (uint32_t w = 1; w < NW; w++) sum += red[ci & 1][w][t][nn];
                const uint32_t row = it.r0 + nn;
                if (row < it.r1) {
                    const size_t o = (size_t)t * ldy + row;
                    const float v = !resid ? sum
                                    : coh  ? __hip_atomic_load(resid + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + sum
                                           : resid[o] + sum;
                    __hip_atomic_store(y + o, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            // the stores acknowledged, then the item counted; the count that
            // completes the step sets its ready flags (a step no later step
            // waits for is not counted)
            if (stp->count) {
                __builtin_amdgcn_s_waitcnt(0);
                if (lane == 0 &&
                    __hip_atomic_fetch_add(ctr(p.done, it.step), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        stp->items - 1) {
                    for (uint32_t c2 = 0; c2 < kChainFlags; c2++)
                        __hip_atomic_store(ctr(p.ready, it.step * kChainFlags + c2), 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        // ---- the last workgroup out returns the counters and flags to
        // zero.  This wavefront has counted every item of its workgroup
        // (its fetch-adds returned), so when the exit count completes, every
        // count of the launch has been made. ----
        uint32_t last = 0;
        if (lane == 0)
            last = __hip_atomic_fetch_add(p.exit_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.nwg - 1;
        if (__builtin_amdgcn_readfirstlane(last)) {
            for (uint32_t t = lane; t < p.nsteps; t += 64)
                __hip_atomic_store(ctr(p.done, t), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (uint32_t f = lane; f < p.nsteps * kChainFlags; f += 64)
                __hip_atomic_store(ctr(p.ready, f), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0) __hip_atomic_store(p.exit_cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (nitems) {
        // ---- a streaming wavefront ----
        // This wavefront's LDS: two A-operand slots and a 16-byte zero slot
        // (as the row-split kernel).
        uint8_t *const wbase = lds + wv * gemv_rows_wave_lds(M);
        const uint32_t tt = mrow & 7, pp = mrow >> 3;
        const bool a_active = tt < M && pp < 3;
        const uint8_t *const arow = a_active ? wbase + ((pp * M + tt) * 2 + hh) * 16 : wbase + 512 * R;
        const uint32_t a_slot = a_active ? 256 * R : 0;
        const uint32_t a_step = a_active ? R * 32 : 0;
        if (lane < 4) reinterpret_cast<uint32_t *>(wbase + 512 * R)[lane] = 0u;

        // ---- load side: item li, its block lb is loaded next ----
        uint32_t li = 0, lb = 0;
        uint32_t l_step = 0, l_n = 1, l_k0 = 0, l_ldx = 1, l_k = 1, l_wait = 0;
        const uint8_t *l_codes = nullptr;   // this lane's row, the wavefront's first K block
        const float *l_sc = nullptr;        // this lane's scale row, the wavefront's first K block
        const float *l_x = nullptr;
        auto load_item = [&](uint32_t idx) {
            const ItemRef it = item_ref(steps, ilist[idx]);
            const StepPtr stp = steps + it.step;
            const uint32_t rl = min(it.r0 + mrow, it.r1 - 1);
            const uint32_t KB = stp->kb;
            l_k0 = wv * KB / NW;
            l_n = (wv + 1) * KB / NW - l_k0;
            l_codes = global_ptr(stp->seg[it.si].codes) +
                      ((size_t)(rl >> 7) * KB * 4 + ((rl >> 5) & 3)) * kSubBytes + hh * 512 + (rl & 31) * 16 +
                      (size_t)l_k0 * kBlockBytes;
            const uint32_t ga = it.r0 >> 7, gb = (it.r1 - 1) >> 7;
            const bool out_in_a = ((it.r0 + mrow) >> 7) == ga;
            l_sc = global_ptr(stp->seg[it.si].scale) + (size_t)(out_in_a ? ga : gb) * KB + l_k0;
            l_x = global_ptr(stp->x);
            l_ldx = stp->ldx;
            l_k = stp->k;
            l_wait = stp->wait;
            l_step = it.step;
        };

        // ---- the ring: slot d holds a block's weights, its scale (this
        // lane's output column) and its activations ----
        u32x4_t buf[DEPTH][4] = {};
        float sc[DEPTH] = {};
        XBlock<MT> xr[DEPTH] = {};
        uint32_t xpend = 0;   // bit d: slot d holds zero stand-ins for its activations
        auto issue = [&](uint32_t d) {
            const uint8_t *src = l_codes + (size_t)lb * kBlockBytes;
#pragma unroll
            for (uint32_t q = 0; q < 4; q++)
                buf[d][q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(src + q * kChunkBytes));
            sc[d] = l_sc[lb];
            // activations only once the step's inputs are known complete
            const bool known = !l_wait || ready >= l_step;
            load_x<MT, COH>(xr[d], known ? l_x : global_ptr(p.zero), known ? l_ldx : 0u, M,
                            known ? l_k : kChainZeroFloats, known ? l_k0 + lb : 0u, lane);
            xpend = known ? xpend & ~(1u << d) : xpend | (1u << d);
            // next block of the list (the last one repeats: loaded, never used)
            if (lb + 1 < l_n) {
                lb++;
            } else if (li + 1 < nitems) {
                li++;
                lb = 0;
                load_item(li);
            }
        };

        // ---- consume side: item ci, its block cb.  The ring starts empty
        // and the loop fills it: the first DEPTH - 1 positions consume the
        // blocks of a stand-in item (ci = -1) nothing was loaded for, whose
        // partials are dropped.  The loop's first positions are then the same
        // code as every later one: a separate fill ahead of the loop left the
        // compiler paths into the loop on which it counted fewer loads in
        // flight, and every block of the loop waited for them. ----
        uint32_t ci = ~0u, cb = 0, c_n = DEPTH - 1, c_step = 0, c_wait = 0, c_k0 = 0, c_k = 1, c_ldx = 1;
        const float *c_x = nullptr;
        auto use_item = [&](uint32_t idx) {
            const uint32_t e = ilist[idx];
            const StepPtr stp = steps + (e >> 16);
            const uint32_t KB = stp->kb;
            c_k0 = wv * KB / NW;
            c_n = (wv + 1) * KB / NW - c_k0;
            c_step = e >> 16;
            c_wait = stp->wait;
            c_x = global_ptr(stp->x);
            c_ldx = stp->ldx;
            c_k = stp->k;
            cb = 0;
        };

        // Entering item ci at ring position d (its first block sits in slot
        // (d + 1) % DEPTH): wait for the outputs of earlier steps if needed,
        // reload the activations the ring holds zero stand-ins for (the
        // item's first DEPTH-1 blocks may be in the ring), stage the first
        // block's.  Returns whether that block was staged shifted.
        auto enter = [&](auto dpos, uint32_t g) -> bool {
            constexpr uint32_t d = decltype(dpos)::value;
            if (c_wait && ready < c_step) wait_steps(c_step);
            uint32_t mine = 0;   // the ring slots holding this item's blocks
#pragma unroll
            for (uint32_t i = 0; i + 1 < DEPTH; i++)
                if (i < c_n) mine |= 1u << ((d + 1 + i) % DEPTH);
            if (xpend & mine) {
                // All reloads issued, then one wait for everything in flight
                // (the ring's loads were issued before the wait for earlier
                // steps and have mostly landed): the reloads' latency is paid
                // once per item, and after the wait no register of this path
                // holds a load in flight, so the compiler's count for the
                // ring's unconditional loads is that of the plain path.
#pragma unroll
                for (uint32_t i = 0; i + 1 < DEPTH; i++) {
                    const uint32_t slot = (d + 1 + i) % DEPTH;
                    if (i < c_n && ((xpend >> slot) & 1u))
                        load_x<MT, COH>(xr[slot], c_x, c_ldx, M, c_k, c_k0 + i, lane);
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
                xpend &= ~mine;
            }
            return stage_xblock<MT>(xr[(d + 1) % DEPTH], wbase + (g & 1) * 256 * R, M, R, c_k, c_k0, lane);
        };

        load_item(0);
        bool wide_cur = false, wide_nxt = false;

        f32x16_t acc = {};
        const f32x16_t zero = {};
        uint32_t g = 0;   // blocks consumed by this wavefront
        // Once the list is done the remaining positions of the pass still
        // issue their loads (of the list's last block again, never used):
        // the loop leaves at its end only, and on every path through it each
        // position issues the same loads, so the compiler counts the loads in
        // flight exactly (positions that skipped their loads on the way out
        // made it count too few before every block).
        bool fin = false;
        while (!fin) {
            static_for<0, DEPTH>([&](auto dc) {
                constexpr uint32_t d = decltype(dc)::value;
                issue((d + DEPTH - 1) % DEPTH);
                if (fin) return;
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t par = g & 1;
                u32x4_t araw[8];
#pragma unroll
                for (uint32_t i = 0; i < 8; i++)
                    araw[i] = *reinterpret_cast<const u32x4_t *>(arow + par * a_slot + i * a_step);
                if (cb + 1 < c_n)
                    wide_nxt = stage_xblock<MT>(xr[(d + 1) % DEPTH], wbase + (par ^ 1) * 256 * R, M, R, c_k,
                                                c_k0 + cb + 1, lane);
                __builtin_amdgcn_sched_barrier(0);
                f32x16_t part;
#pragma unroll
                for (uint32_t jj = 0; jj < 4; jj++)
#pragma unroll
                    for (uint32_t q = 0; q < 2; q++) {
                        const bf16x8_t bop = e4m3x8_to_bf16x8_cvt(buf[d][jj][2 * q], buf[d][jj][2 * q + 1], 1.0f);
                        const bf16x8_t aop = __builtin_bit_cast(bf16x8_t, araw[jj * 2 + q]);
                        part = mfma32x32x16(aop, bop, (jj == 0 && q == 0) ? zero : part);
                    }
                const float scv = wide_cur ? sc[d] * kActUnshift : sc[d];
#pragma unroll
                for (uint32_t r = 0; r < 12; r++)
                    if ((r & 3) < MT) acc[r] = __builtin_fmaf(scv, part[r], acc[r]);
                wide_cur = wide_nxt;
                g++;
                if (++cb < c_n) return;

                // ---- item ci done: the partials to LDS for the fifth
                // wavefront, then the next item ----
                if (ci != ~0u) {
#pragma unroll
                    for (uint32_t r = 0; r < 4; r++) {
                        const uint32_t t = 4 * hh + r;
                        if (t < M) red[ci & 1][wv][t][mrow] = (acc[r] + acc[r + 4]) + acc[r + 8];
                    }
                    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the LDS writes done
                    __builtin_amdgcn_s_barrier();
                }
                acc = zero;
                if (++ci == nitems) {
                    fin = true;
                    return;
                }
                use_item(ci);
                wide_cur = enter(dc, g);
            });
        }
    }
}

namespace {
using ChainKernel = void (*)(ChainParams);
ChainKernel chain_kernel(uint32_t m, bool coh) {
    static const ChainKernel k[2][4] = {
        {gemv_chain_kernel<1, false>, gemv_chain_kernel<2, false>, gemv_chain_kernel<4, false>,
         gemv_chain_kernel<8, false>},
        {gemv_chain_kernel<1, true>, gemv_chain_kernel<2, true>, gemv_chain_kernel<4, true>,
         gemv_chain_kernel<8, true>}};
    return k[coh][m <= 1 ? 0 : m <= 2 ? 1 : m <= 4 ? 2 : 3];
}
}  // namespace

hipError_t launch_chain(const ChainParams &p, hipStream_t stream) {
    if (p.m == 0 || p.m > kGemvMaxM || p.nwg == 0) return hipErrorInvalidValue;
    static bool attr_set = false;
    if (!attr_set) {
        for (bool coh : {false, true})
            for (uint32_t m : {1u, 2u, 4u, 8u}) {
                const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(chain_kernel(m, coh)),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)kChainLds);
                if (e != hipSuccess) return e;
            }
        attr_set = true;
    }
    hipLaunchKernelGGL(chain_kernel(p.m, p.coherent != 0), dim3(p.nwg), dim3(64 * (kChainWaves + 1)), kChainLds,
                       stream, p);
    return hipGetLastError();
}

}  // namespace q35mm
