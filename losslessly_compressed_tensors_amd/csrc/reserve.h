// Block scans over per-block overflow summaries and the arena reservation
// that follows them (one workgroup of 256 threads), shared by the overflow
// bookkeeping launches (compaction.hip) and the fused compress (compress.hip).
//
// Follows LCT/kernels/generic/metadata.py:13-38 (scans) and
// LCT/kernels/tensor_buffer.py:37-91 (reservation).  The per-block values come
// from a source policy: loads of summaries an earlier launch wrote
// (SummaryLoads), or tagged control words that workgroups of the same launch
// publish (PolledSummaries).
#pragma once

#include "allocator.h"

namespace lct {

constexpr int kPrefixPer = 16;   // blocks per thread per pass of SummaryLoads (4096 per pass)

// Exclusive prefix sums of three values over the 256 threads of a block, with
// their totals; one exchange through `scratch` (3 * kWavesPerBlock ints).
// Contains barriers.
__device__ __forceinline__ void block_exclusive_scan3(const int32_t (&v)[3], int32_t *scratch,
                                                      int32_t (&before)[3],
                                                      int32_t (&total)[3]) {
    const int wave = threadIdx.x / kWave;
    int32_t inclusive[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        inclusive[k] = wave_inclusive_scan(v[k]);
        if (wave_lane() == kWave - 1) scratch[k * kWavesPerBlock + wave] = inclusive[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        int32_t prior = 0, sum = 0;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) {
            const int32_t s = scratch[k * kWavesPerBlock + w];
            prior += w < wave ? s : 0;
            sum += s;
        }
        before[k] = prior + inclusive[k] - v[k];
        total[k] = sum;
    }
    __syncthreads();
}

// summaries layout (int32[5*nb + 1]): per-block overflow counts | tail bytes |
// exclusive count scan | exclusive byte scan | list of blocks with overflow |
// list length.  The per-block counts and bytes come from `source` (for
// SummaryLoads, the first two arrays, which an earlier encoder launch wrote);
// this function writes the list, its length, the block metadata
// blocks[3*nb] = {count, first, byte_base}, counts[4] = {entries, tail bytes,
// 0, incomplete} and, with kWriteScans, the two exclusive scans.  Each pass
// covers Source::kPer consecutive blocks per thread (256 * kPer per pass),
// stored as kPer / 4 16-byte buffer accesses per array (blocks past the end
// are not written); running
// totals carry from pass to pass, so any block count gives the same
// deterministic layout (entries in block order, lanes ascending within a
// block).
//
// The reservation is a policy: `reserve.begin(scratch)` runs before the scan
// (a buffered call takes the arena lock and reads its free list there; for
// a source of loads, once the first pass's loads are in flight, so those
// latencies overlap), `reserve.finish(request, scratch, incomplete)` at the
// end.  kWriteScans = false leaves the exclusive scans of summaries[2nb, 4nb)
// unwritten (the block metadata holds the same values).  Returns the totals
// written to counts (the same in every thread).
// Workgroup-wide; contains barriers.
struct ScanTotals {
    int32_t entries;
    int32_t bytes;
    bool incomplete;
};

template <bool kWriteScans, class Source, class Reserve>
__device__ __forceinline__ ScanTotals scan_allocate(Source &source, int32_t *__restrict__ summaries,
                                              int32_t *__restrict__ counts,
                                              int32_t *__restrict__ blocks, int32_t n_blocks,
                                              Reserve &reserve) {
    __shared__ int32_t scratch[3 * kWavesPerBlock];
    constexpr int kPer = Source::kPer;      // blocks per thread per pass
    constexpr int kPass = kPer * kLanes;    // blocks per pass
    const int t = threadIdx.x;
    const int64_t nb = n_blocks;
    const uint32_t bytes = static_cast<uint32_t>(n_blocks) * 4u;
    const __amdgpu_buffer_rsrc_t first_out = make_rsrc(summaries + 2 * nb, bytes);
    const __amdgpu_buffer_rsrc_t base_out = make_rsrc(summaries + 3 * nb, bytes);
    const __amdgpu_buffer_rsrc_t meta_count = make_rsrc(blocks, bytes);
    const __amdgpu_buffer_rsrc_t meta_first = make_rsrc(blocks + nb, bytes);
    const __amdgpu_buffer_rsrc_t meta_base = make_rsrc(blocks + 2 * nb, bytes);
    int32_t *list = summaries + 4 * nb;
    int32_t carry[3] = {0, 0, 0};   // entries, tail bytes, listed blocks
    int32_t c[kPer], v[kPer];
    // A source whose values are in memory (kEarly) has the first pass's loads
    // issued before the arena lock is requested, so their latency and the
    // lock's overlap; a polled source takes the lock first.
    if (Source::kEarly) source.load(0, c, v);
    reserve.begin(scratch);
    for (int base = 0; base < n_blocks; base += kPass) {
        const int32_t first_block = base + t * kPer;
        const uint32_t off = static_cast<uint32_t>(first_block) * 4u;
        const bool whole = first_block + kPer <= n_blocks;
        if (base > 0 || !Source::kEarly) source.load(base, c, v);
        int32_t run[3] = {0, 0, 0};
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            run[0] += c[k];
            run[1] += v[k];
            run[2] += c[k] > 0 ? 1 : 0;
        }
        int32_t before[3], total[3];
        block_exclusive_scan3(run, scratch, before, total);
        int32_t count_before = carry[0] + before[0];
        int32_t byte_before = carry[1] + before[1];
        int32_t list_before = carry[2] + before[2];
        int32_t firsts[kPer], bases[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            firsts[k] = count_before;
            bases[k] = byte_before;
            if (c[k] > 0) list[list_before++] = first_block + k;
            count_before += c[k];
            byte_before += v[k];
        }
        if (!whole) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const uint32_t o = off + 4 * k;
                if (kWriteScans) {
                    __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(firsts[k]), first_out, o, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(bases[k]), base_out, o, 0, 0);
                }
                __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(c[k]), meta_count, o, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(firsts[k]), meta_first, o, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(bases[k]), meta_base, o, 0, 0);
            }
        }
#pragma unroll
        for (int q = 0; whole && q < kPer / 4; ++q) {
            using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;
            const u32x4 fq = {static_cast<uint32_t>(firsts[4 * q]),
                              static_cast<uint32_t>(firsts[4 * q + 1]),
                              static_cast<uint32_t>(firsts[4 * q + 2]),
                              static_cast<uint32_t>(firsts[4 * q + 3])};
            const u32x4 bq = {static_cast<uint32_t>(bases[4 * q]),
                              static_cast<uint32_t>(bases[4 * q + 1]),
                              static_cast<uint32_t>(bases[4 * q + 2]),
                              static_cast<uint32_t>(bases[4 * q + 3])};
            const u32x4 cq = {static_cast<uint32_t>(c[4 * q]), static_cast<uint32_t>(c[4 * q + 1]),
                              static_cast<uint32_t>(c[4 * q + 2]),
                              static_cast<uint32_t>(c[4 * q + 3])};
            if (kWriteScans) {
                __builtin_amdgcn_raw_buffer_store_b128(fq, first_out, off + 16 * q, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(bq, base_out, off + 16 * q, 0, 0);
            }
            __builtin_amdgcn_raw_buffer_store_b128(cq, meta_count, off + 16 * q, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(fq, meta_first, off + 16 * q, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(bq, meta_base, off + 16 * q, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) carry[k] += total[k];
    }
    // A polled source whose summaries did not all arrive leaves the tensor
    // incomplete: counts[3] and the reservation's status say so.
    const bool incomplete = source.incomplete();
    if (t == 0) {
        counts[0] = carry[0];
        counts[1] = carry[1];
        counts[2] = 0;
        counts[3] = incomplete ? 1 : 0;
        summaries[5 * nb] = carry[2];
    }
    // Two metadata bytes per overflowing stream: lane, then start step.
    reserve.finish(carry[1] + 2 * carry[0], scratch, incomplete);
    return ScanTotals{carry[0], carry[1], incomplete};
}

// Per-block overflow counts and tail bytes from summaries[0, nb) and
// summaries[nb, 2nb), written by an earlier launch.  Each pass covers 4096
// blocks, 16 consecutive ones per thread; a thread whose 16 blocks all exist
// moves them with 16-byte accesses, the one that straddles the end (and those
// past it) with 4-byte accesses, which the range check reads as 0.
struct SummaryLoads {
    static constexpr bool kEarly = true;
    static constexpr int kPer = kPrefixPer;
    __amdgpu_buffer_rsrc_t count_in, bytes_in;
    int32_t n_blocks;

    __device__ SummaryLoads(const int32_t *summaries, int32_t nb)
        : count_in(make_rsrc(summaries, static_cast<uint32_t>(nb) * 4u)),
          bytes_in(make_rsrc(summaries + nb, static_cast<uint32_t>(nb) * 4u)), n_blocks(nb) {}

    __device__ void load(int base, int32_t (&c)[kPrefixPer], int32_t (&v)[kPrefixPer]) const {
        const int32_t first_block = base + static_cast<int32_t>(threadIdx.x) * kPrefixPer;
        const uint32_t off = static_cast<uint32_t>(first_block) * 4u;
        if (first_block + kPrefixPer <= n_blocks) {
#pragma unroll
            for (int q = 0; q < kPrefixPer / 4; ++q) {
                const auto cq = __builtin_amdgcn_raw_buffer_load_b128(count_in, off + 16 * q, 0, 0);
                const auto vq = __builtin_amdgcn_raw_buffer_load_b128(bytes_in, off + 16 * q, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    c[4 * q + k] = static_cast<int32_t>(cq[k]);
                    v[4 * q + k] = static_cast<int32_t>(vq[k]);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < kPrefixPer; ++k) {
                c[k] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(count_in, off + 4 * k, 0, 0));
                v[k] = static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b32(bytes_in, off + 4 * k, 0, 0));
            }
        }
    }

    __device__ bool incomplete() const { return false; }
};

// Per-block summaries that the encoding workgroups of the same launch publish
// as tagged control words (kControlPartials + block): each thread polls its
// pass's 16 words until each carries `epoch`, with a sleep between rounds and
// at most `polls` rounds.  A word that does not arrive, or that marks a block
// without a center, counts as 0 and makes the scan incomplete.
struct PolledSummaries {
    static constexpr bool kEarly = false;
    // Four blocks per thread (1024 per pass) keep the polled scan's registers
    // within the encoders' budget: the bookkeeping workgroup shares their
    // kernel, whose register count is the larger of the two paths.
    static constexpr int kPer = 4;
    const uint64_t *control;
    uint32_t epoch;
    int32_t n_blocks;
    int32_t polls;
    bool failed;

    __device__ void load(int base, int32_t (&c)[kPer], int32_t (&v)[kPer]) {
        const int32_t first_block = base + static_cast<int32_t>(threadIdx.x) * kPer;
        const uint64_t *words = control + kControlPartials + first_block;
        uint32_t pending = 0;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            c[k] = 0;
            v[k] = 0;
            if (first_block + k < n_blocks) pending |= 1u << k;
        }
        for (int round = 0; pending != 0 && round <= polls; ++round) {
            if (round > 0) __builtin_amdgcn_s_sleep(8);
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                if ((pending >> k) & 1u) {
                    const uint64_t word = control_load(words + k);
                    if (tagged_with(word, epoch)) {
                        const uint32_t value = static_cast<uint32_t>(word);
                        const uint32_t count = value >> 17;
                        if (count == kFailedBlock) {
                            failed = true;
                        } else {
                            c[k] = static_cast<int32_t>(count);
                            v[k] = static_cast<int32_t>(value & 0x1FFFFu);
                        }
                        pending &= ~(1u << k);
                    }
                }
            }
        }
        if (pending != 0) failed = true;
    }

    // Whether any thread saw a failure (uniform).  Contains barriers.  A
    // ballot per wave and one LDS word per wave: HIP's __syncthreads_or
    // brings 256 bytes of library LDS into every kernel that scans, which
    // leaves the encoder at W = 19 one workgroup per CU short (LDS is
    // granted in 1280-byte steps, and five workgroups need <= 32000 bytes).
    __device__ bool incomplete() const {
        __shared__ int32_t any[kWavesPerBlock];
        const bool wave_failed = __ballot(failed) != 0;
        if (wave_lane() == 0) any[threadIdx.x / kWave] = wave_failed ? 1 : 0;
        __syncthreads();
        int32_t seen = 0;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) seen |= any[w];
        __syncthreads();   // `any` may be rewritten by the next call
        return seen != 0;
    }
};

// No arena: the scans only (private storage, whose exact-size arrays the host
// allocates from counts).
struct NoReserve {
    __device__ void begin(int32_t *) {}
    __device__ void finish(int32_t, int32_t *, bool) {}
};

// lct_prefix_allocate's reservation: the lock, then the free list in
// registers (allocator_begin / allocator_finish); nothing when not buffered.
struct RegisterReserve {
    AllocatorMeta meta;
    int32_t *descriptor;
    int32_t *flag;   // one LDS int
    bool active;
    AllocatorSnapshot snap;

    __device__ void begin(int32_t *) {
        if (active) allocator_begin(meta, snap, flag);
    }
    __device__ void finish(int32_t request, int32_t *scratch, bool) {
        if (active) allocator_finish(meta, snap, request, descriptor, scratch, true);
    }
};

// lct_allocate_compact's reservation (workgroup 0).  begin: thread 0 reads
// the lock word while the first pass's loads and the pending descriptors'
// values are in flight; then, with the lock seen free at version v, thread 0
// takes it (v -> v + 1) while every thread reads the free list into LDS with
// agent-scope loads: the copy is current exactly when that compare-and-swap
// succeeds (otherwise the lock is waited for and the list read again).  The
// deferred frees then run on the LDS copy, in order.  finish: the first-fit
// reservation on the LDS copy, the list written back, the descriptor, and the
// lock to v + 2 after a release.  kPublishAll: an agent-scope release fence
// that publishes every write of the workgroup (lct_allocate_compact's waiters
// then read the metadata in the same launch); without it only the free list
// must be visible before the lock (everything else is read by later launches),
// so the list is written back with agent-scope atomic stores and the release
// is a wait for those stores -- the fence's write-back of this XCD's whole L2,
// which holds the encoders' payload, took 2.5 us at 4096 blocks.  Two memory round trips before the scan, where the
// register path takes three (lock, fence, list) plus one per free.
template <bool kPublishAll>
struct LdsReserve {
    AllocatorMeta meta;
    int32_t *descriptor;
    lct_pending_frees frees;
    int32_t *list;   // LDS int32[2 * regions]: starts, then sizes
    LdsFreeList f;
    int32_t held;

    __device__ void read_list(int32_t *shared) {
        const int32_t regions = meta.regions;
        for (int32_t i = threadIdx.x; i < regions; i += kLanes) {
            list[i] = coherent_load(meta.starts + i);
            list[regions + i] = coherent_load(meta.sizes + i);
        }
        if (threadIdx.x == 0) {
            shared[2] = coherent_load(meta.count);
            shared[3] = coherent_load(meta.generation);
        }
    }

    __device__ void begin(int32_t *scratch) {
        __shared__ int32_t shared[4];   // seen version, held version, count, generation
        __shared__ int32_t pending[LCT_MAX_PENDING_FREES][4];
        const int t = threadIdx.x;
        if (t == 0) shared[0] = coherent_load(meta.lock);
#pragma unroll
        for (int j = 0; j < LCT_MAX_PENDING_FREES; ++j)
            if (j < frees.count && t < 4) pending[j][t] = frees.descriptor[j][t];
        __syncthreads();
        const int32_t seen = shared[0];
        if ((seen & 1) == 0) {
            if (t == 0) {
                int32_t expected = seen;
                shared[1] = __hip_atomic_compare_exchange_strong(
                                meta.lock, &expected, seen + 1, __ATOMIC_ACQUIRE,
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                ? seen
                                : -1;
            }
            read_list(shared);
        } else if (t == 0) {
            shared[1] = -1;
        }
        __syncthreads();
        held = shared[1];
        if (held < 0) {
            if (t == 0) shared[1] = take_lock_thread0(meta.lock, -1, meta.spins);
            __syncthreads();
            held = shared[1];
            if (held >= 0) read_list(shared);
            __syncthreads();
        }
        f = LdsFreeList{list, list + meta.regions, meta.regions, shared[2], shared[3]};
        if (held < 0) return;
#pragma unroll
        for (int j = 0; j < LCT_MAX_PENDING_FREES; ++j) {
            if (j < frees.count) {
                const int32_t d[4] = {pending[j][0], pending[j][1], pending[j][2], pending[j][3]};
                if (lds_free(f, d, scratch) == kStatusOk) {
                    if (t == 0) {
                        __hip_atomic_store(frees.descriptor[j] + 2, kStatusFreed, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                        // A later copy of the same descriptor now reads as
                        // freed, so a second free of it is rejected, as the
                        // immediate free would reject it (status 4).
#pragma unroll
                        for (int k = j + 1; k < LCT_MAX_PENDING_FREES; ++k)
                            if (k < frees.count && frees.descriptor[k] == frees.descriptor[j])
                                pending[k][2] = kStatusFreed;
                    }
                    __syncthreads();
                }
            }
        }
    }

    int32_t status;   // the reservation's status (uniform after finish)

    __device__ void finish(int32_t request, int32_t *scratch, bool incomplete) {
        const int t = threadIdx.x;
        // An incomplete scan (summaries that did not arrive) gives status 7
        // whatever the reservation did, since its request may be short: a
        // region it reserved is held (and freed) like any other.
        int32_t outcome;
        if (held < 0) {
            outcome = kStatusLock;
            if (t == 0) {
                descriptor[0] = -1;
                descriptor[1] = 0;
                descriptor[3] = -1;
            }
        } else {
            int32_t out[3];
            lds_reserve(f, request, scratch, out);
            if (kPublishAll)
                lds_write_back(f, meta);
            else
                lds_write_back_coherent(f, meta);
            outcome = out[2];
            if (t == 0) {
                descriptor[0] = out[0];
                descriptor[1] = out[1];
                descriptor[3] = f.generation;
            }
        }
        status = incomplete ? kStatusIncomplete : outcome;
        if (t == 0) {
            descriptor[2] = status;
            const int32_t bits = failure_bits(outcome, request) | (incomplete ? kFailIncomplete : 0);
            if (bits != 0) record_failure(meta, bits);
        }
        if (kPublishAll) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        } else {
            // The free list's agent-scope stores have completed (vmcnt 0) before
            // any thread passes the barrier; the compiler keeps them above it.
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
        }
        __syncthreads();
        if (held >= 0 && t == 0)
            __hip_atomic_store(meta.lock, held + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
};

// The arena reservation of one tensor of a batched launch (compress or
// fused update).  The batch's deferred frees belong to job 0, whose bookkeeping applies them right after it takes the
// lock and then posts `gate`; the other jobs' bookkeeping waits for that word
// (bounded) before it asks for the lock, so every reservation of the batch
// follows the frees, as the reservations of consecutive single launches would.
// Job 0 is dispatched first and waits for nothing of the later jobs.  A gate
// that does not arrive marks the tensor incomplete.  gate == nullptr (no
// frees): plain LdsReserve.
struct GatedReserve {
    LdsReserve<false> inner;
    uint64_t *gate;
    bool post;
    uint32_t epoch;
    int32_t polls;
    bool late;

    __device__ void begin(int32_t *scratch) {
        __shared__ int32_t arrived;
        if (gate != nullptr && !post) {
            if (threadIdx.x == 0) {
                uint64_t word = control_load(gate);
                for (int i = 0; !tagged_with(word, epoch) && i < polls; ++i) {
                    __builtin_amdgcn_s_sleep(8);
                    word = control_load(gate);
                }
                arrived = tagged_with(word, epoch) ? 1 : 0;
            }
            __syncthreads();
            late = arrived == 0;
        }
        inner.begin(scratch);
        if (gate != nullptr && post && threadIdx.x == 0) control_store(gate, tagged_word(epoch, 1));
    }

    __device__ void finish(int32_t request, int32_t *scratch, bool incomplete) {
        inner.finish(request, scratch, incomplete || late);
    }
};

}  // namespace lct
