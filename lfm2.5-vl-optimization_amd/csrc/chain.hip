// A chain of batch-1 weight-only INT8 GEMVs (a decode step's linears) as one persistent launch on gfx950.
//
// Op j of the chain is y_j = epi(x_j W_j^T s_j) (plain, SwiGLU over w1|w3, or residual add into y_j), and op j may
// read anything ops 0 .. j-1 wrote: op j's math starts only once every output of op j - 1 is written. Launched as
// separate kernels, each GEMV pays a kernel boundary and then its first HBM round trip before any weight arrives
// (~1.6 us + ~2 us for a 4-34 MB matrix). Here the weights -- which never depend on an earlier op -- are streamed
// continuously across op boundaries, and only the activations wait for the dependency. (Measured on MI355X, each op
// boundary still costs about 3 us -- flag seen ~0.7 us after it lands, inputs staged ~1 us, outputs stored ~0.5 us,
// all device-coherent round trips to the memory side -- so a whole LFM2-1.2B decode step runs slower as one chain
// than as separate kernels replayed from one HIP graph; it is on a par with separate eager launches.)
//
//   * One workgroup per CU (grid = CU count, every workgroup resident at once), output rows of each op split evenly
//     over the workgroups, whole rows dealt round-robin to the 8 compute wavefronts of a workgroup.
//   * Each compute wavefront streams its rows' weights, 1 KiB (16 bytes per lane) per load, straight into a private
//     ring of 16 LDS slots with buffer_load_dwordx4 ... nt lds, running up to 16 KiB ahead of its math, across op
//     boundaries (128 KiB per CU, 32 MiB over the chip). Its vector memory counter tracks nothing but the ring, so
//     "the next B slots have landed" is a constant s_waitcnt vmcnt(16 - B) before every item of B slots; after the
//     item's math the B slots are refilled.
//   * A ninth wavefront does all other memory traffic: it waits for the previous op (below), stages x_j, the
//     scales and the residual rows of the workgroup's outputs into LDS, and after the compute wavefronts are done
//     stores the outputs and publishes the op's completion.
//   * Completion: workgroup g writes its outputs with device-coherent stores (sc1, written through to the memory
//     side), waits for them (s_waitcnt vmcnt(0)), then stores flag[g] = epoch(j) into each of 8 copies of the flag
//     array. A waiter polls the flags of all workgroups in copy g % 8 with device-coherent loads until each has
//     reached epoch(j) -- with one copy, 256 pollers on the same 8 cache lines queue at one memory channel -- and
//     reads every input of op j + 1 with device-coherent loads. No cache-wide writeback or invalidate, no
//     read-modify-write atomics.
//   * epoch(j) = gen * 1024 + j + 1 for the gen-th launch on a workspace (gen is read at the start, incremented
//     once all workgroups have read it), compared as a wrapping difference, so the flags never need resetting.
//     Every wait is bounded (20 ms of the real-time counter by default, knob LFM2Q_CHAIN_WAIT_MS): a wait that runs
//     out writes the launch's tag gen + 1 into the workspace's error word, and from then on every wait of every
//     workgroup of that launch returns at once, so the kernel always finishes. The next launch has another tag, so
//     its waits are not cut short by an earlier launch's error.
//
// Per row the arithmetic is exactly the batch-1 GEMV kernels' (gemv_math.hpp: lane l owns 16-byte chunk l + 64 u of
// the row, chunk products on v_dot2_f32_bf16 in order of u, fold_sum over the lanes, the same epilogue), so each
// output is bit-identical to the separate lfm2q_gemv_w8 / _swiglu / _residual call on the same inputs.
//
// Reference: the reference overlaps consecutive decode GEMVs with programmatic dependent launch
// (kernels/lfm2_decode.cu:24-62): a kernel prefetches its weights before griddepcontrol.wait (:500-512, :600-609).
#include "common.hpp"
#include "gemv_math.hpp"
#include "status.hpp"

#include <algorithm>
#include <atomic>

namespace lfm2q {
namespace {

#ifndef LFM2Q_CHAIN_CW
#define LFM2Q_CHAIN_CW 8
#endif
constexpr int CW = LFM2Q_CHAIN_CW;    // compute wavefronts per workgroup (two per SIMD)
constexpr int SLOTS = 128 / CW;       // 1 KiB ring slots per compute wavefront: 128 KiB of ring per workgroup
constexpr int UNIT = 1024;            // bytes per slot: one wavefront load, 16 bytes per lane
constexpr int MAX_K = 8192;
constexpr int MAX_ROWS = 512;         // output rows of one op per workgroup
constexpr int MAX_OPS = 128;          // ops per launch (the op table lives in LDS)
constexpr uint32_t EPOCHS = 1024;
constexpr int MAX_G = 1024;           // workgroups (= CUs)
constexpr int WS_GEN = 0, WS_ERR = 1; // workspace words; the flags start 128 bytes in
constexpr int WS_FLAGS = 32;
constexpr int FLAG_COPIES = 8;        // every flag is written to 8 copies of the flag array; workgroup g polls copy g % 8
constexpr int FLAG_STRIDE = 1088;     // words between copies (4352 bytes: the copies sit in different memory channels)
constexpr uint64_t TICKS_PER_MS = 100000;  // the s_memrealtime clock runs at 100 MHz
constexpr int AUX_SC1 = 16;           // device-scope coherent access (sc1)

struct ChainOp {
    const int8_t *W;
    const float *scale;
    const uint16_t *x;
    uint16_t *y;
    int N, K, epi, reserved;
};
static_assert(sizeof(ChainOp) == sizeof(lfm2q_gemv_op), "descriptor layout");
static_assert(FLAG_STRIDE >= MAX_G && CW * SLOTS * UNIT == 128 * 1024, "workspace and ring layout");

struct Lds {
    uint8_t ring[CW][SLOTS][UNIT];  // 128 KiB
    ChainOp ops[MAX_OPS];           // the op table (6 KiB)
    uint16_t xs[MAX_K];             // x_j
    float sc[2][MAX_ROWS];          // scales of the workgroup's rows (w1, w3 for SwiGLU)
    uint16_t hs[MAX_ROWS];          // residual rows (epi 2)
    uint16_t outs[MAX_ROWS];        // results, stored by the sync wavefront
};

// rows [r0, r1) of an op of N rows for workgroup g of G (g N < 2^31: N <= 512 G, G <= 1024, checked on the host)
__device__ __forceinline__ void rows_of(int N, int g, int G, int &r0, int &r1) {
    r0 = (int)((uint32_t)(g * N) / (uint32_t)G);
    r1 = (int)((uint32_t)((g + 1) * N) / (uint32_t)G);
}

// a pointer read from LDS as a wavefront-uniform (scalar) value; readfirstlane returns int, so each half goes
// back through uint32_t before widening (a sign-extended low half would corrupt the address)
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<T *>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Device-coherent accesses through a buffer resource.
__device__ __forceinline__ v4u ld_dev16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX_SC1));
}
__device__ __forceinline__ uint16_t ld_dev2(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, AUX_SC1);
}
__device__ __forceinline__ void st_dev2(uint16_t v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, (int)off, 0, AUX_SC1);
}

// The weight stream of one compute wavefront: op by op, the wavefront's items t = w, w + CW, ... (local indices,
// item t = row row0 + t), per item its NROW weight rows (that row, and S + it for SwiGLU), per row its K / 1024 units. Every member is
// wavefront-uniform (scalar registers); past the last op every load reads zeros through an empty range.
struct Loader {
    const ChainOp *ops;  // the LDS copy
    int n_ops, g, G, w;
    int j;
    v4i desc;
    uint32_t rowb;
    int cpl, nrow, S, row0, t, t_end, r, u;

    __device__ __forceinline__ void open(int from) {
        for (j = from; j < n_ops; ++j) {
            const int N = __builtin_amdgcn_readfirstlane(ops[j].N);
            int r1;
            rows_of(N, g, G, row0, r1);
            t = w;  // local item index; its row is row0 + t
            t_end = r1 - row0;
            if (t < t_end) {
                const int K = __builtin_amdgcn_readfirstlane(ops[j].K);
                nrow = __builtin_amdgcn_readfirstlane(ops[j].epi) == EPI_SWIGLU ? 2 : 1;
                S = N;
                rowb = (uint32_t)K;
                cpl = K / UNIT;
                r = u = 0;
                desc = make_desc(uniform_ptr(ops[j].W), (uint32_t)(nrow * N) * rowb);
                return;
            }
        }
        // past the last op: an empty range over a valid base (the last op's weights), so every load reads zeros
        // without touching memory
        desc = make_desc(uniform_ptr(ops[n_ops - 1].W), 0u);
    }
    __device__ __forceinline__ uint32_t offset() const {
        return j < n_ops ? (uint32_t)(r ? S + row0 + t : row0 + t) * rowb + (uint32_t)u * UNIT : 0u;
    }
    __device__ __forceinline__ void advance() {
        if (j >= n_ops) return;
        if (++u < cpl) return;
        u = 0;
        if (++r < nrow) return;
        r = 0;
        t += CW;
        if (t < t_end) return;
        open(j + 1);
    }
    __device__ __forceinline__ void issue(void *slot, int lane) {
        // the resource must reach the instruction in scalar registers (an asm operand is not moved there by itself)
        const v4i d = {__builtin_amdgcn_readfirstlane(desc[0]), __builtin_amdgcn_readfirstlane(desc[1]),
                       __builtin_amdgcn_readfirstlane(desc[2]), __builtin_amdgcn_readfirstlane(desc[3])};
        // non-temporal: each weight byte is read once (measured: 6.2 -> 7.0 TB/s for a streaming ring like this one)
        asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dwordx4 %0, %1, 0 offen nt lds"
                     ::"v"((uint32_t)lane * 16u + offset()), "s"(d), "{m0}"(lds_addr(slot))
                     : "memory");
    }
    // the next n units of the stream into the ring slots from position p on (a loop, not unrolled: one copy of
    // advance() per call site)
    __device__ __forceinline__ void issue_n(Lds &L, uint32_t p, int n, int lane);
};

__device__ __forceinline__ void Loader::issue_n(Lds &L, uint32_t p, int n, int lane) {
#pragma nounroll
    for (int b = 0; b < n; ++b) {
        issue(L.ring[w][(p + b) & (SLOTS - 1)], lane);
        advance();
    }
}

// One op's items of a compute wavefront: items t = w, w + CW, ... < cnt (local indices; item t is output row
// row0 + t), each NROW weight rows of CPL units. Before an item its B = NROW CPL slots are waited for and read; after
// its math they are refilled with the next B units of the stream. The row sums are reduced on their own (fold_sum
// over one value, or the w1 / w3 pair), which pairs the lanes exactly as the batch-1 GEMV kernels do, so the bits
// are theirs.
template <int CPL, int NROW>
__device__ __forceinline__ void chain_items(Lds &L, Loader &ld, uint32_t &pos, int lane, int w, int cnt, int epi) {
    using D = PairDot<int8_t>;
    constexpr int B = NROW * CPL;
    static_assert(B <= SLOTS, "an item fits the ring");
    v4i xr[CPL][2];
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
        for (int q = 0; q < 2; ++q) xr[u][q] = *reinterpret_cast<const v4i *>(&L.xs[(lane + 64 * u) * 16 + 8 * q]);
    for (int t = w; t < cnt; t += CW) {
        v4i c[B];
        wait_vm<SLOTS - B>();  // units pos .. pos + B - 1 have landed (every earlier refill has been issued)
#pragma unroll
        for (int b = 0; b < B; ++b) c[b] = *reinterpret_cast<const v4i *>(&L.ring[w][(pos + b) & (SLOTS - 1)][16 * lane]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slots are read before they refill
        const uint32_t p = pos;
        pos += B;
        float a[NROW];
#pragma unroll
        for (int rr = 0; rr < NROW; ++rr) {
            a[rr] = 0.f;
#pragma unroll
            for (int u = 0; u < CPL; ++u) a[rr] = D::dot(c[rr * CPL + u], xr[u], a[rr]);
        }
        const float rs = fold_sum<NROW>(a);  // NROW 2: w1 sum in lanes 0-31, w3 sum in lanes 32-63
        if (NROW == 2) {
            const float ru = __uint_as_float(
                __builtin_amdgcn_permlane32_swap(__float_as_uint(rs), __float_as_uint(rs), false, false)[1]);
            if (lane == 0) L.outs[t] = gemv_epilogue<EPI_SWIGLU>(rs, L.sc[0][t], ru, L.sc[1][t], 0u, true);
        } else if (lane == 0) {
            L.outs[t] = epi == EPI_RESIDUAL ? gemv_epilogue<EPI_RESIDUAL>(rs, L.sc[0][t], 0.f, 1.f, L.hs[t], true)
                                            : gemv_epilogue<EPI_NONE>(rs, L.sc[0][t], 0.f, 1.f, 0u, true);
        }
        ld.issue_n(L, p, B, lane);
    }
}

__device__ __forceinline__ void chain_op(Lds &L, Loader &ld, uint32_t &pos, int lane, int w, int cnt, int cpl,
                                         int epi) {
    if (epi == EPI_SWIGLU) {
        switch (cpl) {
            case 1: chain_items<1, 2>(L, ld, pos, lane, w, cnt, epi); break;
            case 2: chain_items<2, 2>(L, ld, pos, lane, w, cnt, epi); break;
            case 4: chain_items<4, 2>(L, ld, pos, lane, w, cnt, epi); break;
            default: chain_items<8, 2>(L, ld, pos, lane, w, cnt, epi); break;
        }
    } else {
        switch (cpl) {
            case 1: chain_items<1, 1>(L, ld, pos, lane, w, cnt, epi); break;
            case 2: chain_items<2, 1>(L, ld, pos, lane, w, cnt, epi); break;
            case 4: chain_items<4, 1>(L, ld, pos, lane, w, cnt, epi); break;
            default: chain_items<8, 1>(L, ld, pos, lane, w, cnt, epi); break;
        }
    }
}

// The workspace words are read and written as relaxed agent-scope atomics: device-coherent accesses (sc1) that the
// compiler neither merges nor moves out of a polling loop (plain loads of one address in a loop with no store would
// be folded into one).
__device__ __forceinline__ uint32_t ld_word(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every workgroup's flag has reached `target`, or the error word is set, or the bound runs out (which
// sets the error word). Lane l reads flags l, l + 64, ... Up to 256 workgroups two polls are in flight, so a
// completed dependency is seen about one memory round trip after its last flag lands; the error word and the clock
// are checked every 8 rounds. Ends with a compiler barrier: the op's input loads are not moved above the wait.
__device__ __forceinline__ bool all_reached(const uint32_t (&f)[4], int lane, int G, uint32_t target) {
    bool ok = true;
#pragma unroll
    for (int e = 0; e < 4; ++e) ok = ok && (lane + 64 * e >= G || (int)(f[e] - target) >= 0);
    return __builtin_amdgcn_ballot_w64(!ok) == 0;
}
// The error word holds the tag (gen + 1) of the last launch whose wait ran out: a later launch on the workspace
// compares it with its own tag, so one expired launch does not cut short the waits of the next.
__device__ __forceinline__ void wait_flags(uint32_t *ws, int G, uint32_t target, int lane, uint32_t tag,
                                           uint64_t wait_ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const uint32_t *flags = ws + WS_FLAGS + (blockIdx.x % FLAG_COPIES) * FLAG_STRIDE;
    if (G <= 256) {
        uint32_t a[4], b[4];
        auto poll = [&](uint32_t(&f)[4]) {
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = lane + 64 * e < G ? ld_word(flags + lane + 64 * e) : 0u;
        };
        poll(a);
        poll(b);
        for (int it = 0;; ++it) {
            if (all_reached(a, lane, G, target)) break;
            if (wait_ticks == 0) {  // a zero bound: a dependency not met at the first poll has run out
                if (lane == 0) st_word(ws + WS_ERR, tag);
                break;
            }
            poll(a);
            if (all_reached(b, lane, G, target)) break;
            poll(b);
            if ((it & 7) == 7) {
                if (ld_word(ws + WS_ERR) == tag) break;
                if (__builtin_amdgcn_s_memrealtime() - t0 > wait_ticks) {
                    if (lane == 0) st_word(ws + WS_ERR, tag);
                    break;
                }
            }
        }
    } else {
        for (;;) {
            bool ok = true;
            for (int i = lane; i < G; i += 64) ok = ok && (int)(ld_word(flags + i) - target) >= 0;
            if (__builtin_amdgcn_ballot_w64(!ok) == 0 || ld_word(ws + WS_ERR) == tag) break;
            if (wait_ticks == 0 || __builtin_amdgcn_s_memrealtime() - t0 > wait_ticks) {
                if (lane == 0) st_word(ws + WS_ERR, tag);
                break;
            }
        }
    }
    asm volatile("" ::: "memory");
}

__global__ __launch_bounds__(64 * (CW + 1)) void gemv_chain_kernel(const ChainOp *__restrict__ ops, int n_ops,
                                                                   uint32_t *__restrict__ ws, int G,
                                                                   uint32_t *__restrict__ status,
                                                                   uint64_t wait_ticks) {
    __shared__ __attribute__((aligned(1024))) Lds L;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = blockIdx.x;
    // the op table into LDS, before any wavefront starts its loads
    for (int i = threadIdx.x; i < n_ops * (int)(sizeof(ChainOp) / 16); i += blockDim.x)
        reinterpret_cast<v4i *>(L.ops)[i] = reinterpret_cast<const v4i *>(ops)[i];
    __syncthreads();

    if (w == CW) {  // ------------------------------------------------------------------ the sync wavefront
        const uint32_t gen = __builtin_amdgcn_readfirstlane(ld_word(ws + WS_GEN));
        for (int j = 0; j < n_ops; ++j) {
            if (j) wait_flags(ws, G, gen * EPOCHS + (uint32_t)j, lane, gen + 1u, wait_ticks);  // op j - 1 done
            const int N = __builtin_amdgcn_readfirstlane(L.ops[j].N), K = __builtin_amdgcn_readfirstlane(L.ops[j].K);
            const int epi = __builtin_amdgcn_readfirstlane(L.ops[j].epi);
            const float *scale = uniform_ptr(L.ops[j].scale);
            int r0, r1;
            rows_of(N, g, G, r0, r1);
            const int nr = r1 - r0;
            // every input of op j into LDS with all its loads in flight at once (one wait): x and the residual rows
            // through device-coherent register loads (an earlier op may have written them), the scales of the
            // workgroup's rows (never written by an op) straight into LDS
            const rsrc_t xr = make_rsrc(uniform_ptr(L.ops[j].x), (uint32_t)K * 2u);
            v4u xv[MAX_K * 2 / 1024];
#pragma unroll
            for (int q = 0; q < MAX_K * 2 / 1024; ++q)
                if (1024 * q < K * 2) xv[q] = ld_dev16(xr, (uint32_t)(1024 * q + 16 * lane));
            const v4i sd = make_desc(scale, (uint32_t)(epi == EPI_SWIGLU ? 2 * N : N) * 4u);
            for (int i = 0; i < nr; i += 64) {
                asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dword %0, %1, 0 offen lds"
                             ::"v"((uint32_t)(r0 + i + lane) * 4u), "s"(sd), "{m0}"(lds_addr(&L.sc[0][i]))
                             : "memory");
                if (epi == EPI_SWIGLU)
                    asm volatile(LFM2Q_LDS_DMA_WAIT "buffer_load_dword %0, %1, 0 offen lds"
                                 ::"v"((uint32_t)(N + r0 + i + lane) * 4u), "s"(sd), "{m0}"(lds_addr(&L.sc[1][i]))
                                 : "memory");
            }
            const rsrc_t yr = make_rsrc(uniform_ptr(L.ops[j].y), (uint32_t)N * 2u);
            if (epi == EPI_RESIDUAL) {  // all row loads issued before the first LDS write
                uint16_t hv[MAX_ROWS / 64];
#pragma unroll
                for (int q = 0; q < MAX_ROWS / 64; ++q)
                    if (64 * q < nr) hv[q] = ld_dev2(yr, (uint32_t)(r0 + 64 * q + lane) * 2u);
#pragma unroll
                for (int q = 0; q < MAX_ROWS / 64; ++q)
                    if (64 * q < nr) L.hs[64 * q + lane] = hv[q];
            }
#pragma unroll
            for (int q = 0; q < MAX_K * 2 / 1024; ++q)
                if (1024 * q < K * 2)
                    *reinterpret_cast<v4u *>(reinterpret_cast<uint8_t *>(L.xs) + 1024 * q + 16 * lane) = xv[q];
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            wg_barrier();  // A_j: op j's inputs are in LDS
            wg_barrier();  // B_j: op j's outputs are in LDS
            for (int i = lane; i < nr; i += 64) st_dev2(L.outs[i], yr, (uint32_t)(r0 + i) * 2u);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the outputs are written before the flag
            if (lane < FLAG_COPIES) st_word(ws + WS_FLAGS + lane * FLAG_STRIDE + g, gen * EPOCHS + (uint32_t)j + 1u);
        }
        if (g == 0) {  // once every workgroup is past the last op (so has read gen), advance gen for the next launch
            wait_flags(ws, G, gen * EPOCHS + (uint32_t)n_ops, lane, gen + 1u, wait_ticks);
            if (lane == 0) st_word(ws + WS_GEN, gen + 1u);
            // every workgroup has stored its last flag, so any expired wait has set the error word by now
            if (lane == 0 && status) st_word(status, ld_word(ws + WS_ERR) == gen + 1u ? 1u : 0u);
        }
        return;
    }

    // ------------------------------------------------------------------------------------ compute wavefronts
    Loader ld{L.ops, n_ops, g, G, w, 0, {}, 0u, 0, 0, 0, 0, 0, 0, 0, 0};
    ld.open(0);
    ld.issue_n(L, 0u, SLOTS, lane);
    uint32_t pos = 0;  // next stream position to consume; pos + SLOTS have been issued
    for (int j = 0; j < n_ops; ++j) {
        wg_barrier();  // A_j
        const int N = __builtin_amdgcn_readfirstlane(L.ops[j].N), epi = __builtin_amdgcn_readfirstlane(L.ops[j].epi);
        const int cpl = __builtin_amdgcn_readfirstlane(L.ops[j].K) / UNIT;
        int r0, r1;
        rows_of(N, g, G, r0, r1);
        chain_op(L, ld, pos, lane, w, r1 - r0, cpl, epi);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // outs written
        wg_barrier();  // B_j
    }
    wait_vm<0>();  // the ring's trailing loads (empty ranges past the last op) before the wavefront ends
}

int check_op(const lfm2q_gemv_op &o, int j, int G) {
    LFM2Q_REQUIRE(o.W && o.scale && o.x && o.y, LFM2Q_ERR_ARG, "gemv_chain: op %d: null pointer", j);
    LFM2Q_REQUIRE(o.epi >= 0 && o.epi <= 2, LFM2Q_ERR_ARG,
                  "gemv_chain: op %d: epi must be 0 (none), 1 (SwiGLU) or 2 (residual), got %d", j, o.epi);
    LFM2Q_REQUIRE(o.K >= UNIT && o.K <= MAX_K && (o.K & (o.K - 1)) == 0, LFM2Q_ERR_SHAPE,
                  "gemv_chain: op %d: K must be 1024, 2048, 4096 or 8192 (K=%d)", j, o.K);
    LFM2Q_REQUIRE(o.N >= 1 && (o.N + G - 1) / G <= MAX_ROWS, LFM2Q_ERR_SHAPE,
                  "gemv_chain: op %d: N must be in [1, %d] (N=%d)", j, MAX_ROWS * G, o.N);
    LFM2Q_REQUIRE((long)(o.epi == 1 ? 2 : 1) * o.N * o.K < (1L << 31), LFM2Q_ERR_SHAPE,
                  "gemv_chain: op %d: W must be smaller than 2 GiB", j);
    LFM2Q_REQUIRE(aligned16(o.W) && aligned16(o.x) && ((uintptr_t)o.y & 1) == 0 && ((uintptr_t)o.scale & 3) == 0,
                  LFM2Q_ERR_ALIGN, "gemv_chain: op %d: W and x must be 16-byte aligned", j);
    return LFM2Q_OK;
}

}  // namespace
}  // namespace lfm2q

using namespace lfm2q;

namespace lfm2q {
namespace {

constexpr int WS_WORDS = WS_FLAGS + FLAG_COPIES * FLAG_STRIDE;

// The checks every chain launch makes (G: the grid, one workgroup per CU).
int check_chain(const char *who, const lfm2q_gemv_op *ops, int n_ops, int &G) {
    G = device_cus();
    LFM2Q_REQUIRE(G >= 1 && G <= MAX_G, LFM2Q_ERR_DEVICE, "%s: %d compute units (at most %d)", who, G, MAX_G);
    for (int j = 0; j < n_ops; ++j)
        if (int st = check_op(ops[j], j, G)) return st;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_chain_kernel, 64 * (CW + 1), 0) != hipSuccess ||
        per_cu < 1)
        return set_error(LFM2Q_ERR_DEVICE, "%s: the kernel does not fit a compute unit", who);
    return LFM2Q_OK;
}

int launch_chain(const char *who, const lfm2q_gemv_op *ops_dev, int n_ops, int G, uint32_t *ws, uint32_t *status,
                 hipStream_t stream) {
    const uint64_t ticks = (uint64_t)std::max(0, knob_int(KNOB_CHAIN_WAIT_MS, 20)) * TICKS_PER_MS;
    gemv_chain_kernel<<<G, 64 * (CW + 1), 0, stream>>>(reinterpret_cast<const ChainOp *>(ops_dev), n_ops, ws, G,
                                                       status, ticks);
    return launch_status(who);
}

// The workspace of lfm2q_gemv_chain_noalloc: one copy per GPU, in the library's own device memory, held until the
// process ends. In host code `scratch` names only a host-side stand-in; the device address comes from
// hipGetSymbolAddress, looked up once per device (with that device current) and kept in scratch_dev.
static __device__ __align__(256) uint32_t scratch[WS_WORDS];
constexpr int MAX_DEVICES = 64;
std::atomic<uint32_t *> scratch_dev[MAX_DEVICES];

int scratch_of_current_device(uint32_t **out) {
    int dev = -1;
    const hipError_t de = hipGetDevice(&dev);
    LFM2Q_REQUIRE(de == hipSuccess && dev >= 0 && dev < MAX_DEVICES, LFM2Q_ERR_DEVICE,
                  "gemv_chain_noalloc: no current device below %d (%s)", MAX_DEVICES, hipGetErrorString(de));
    uint32_t *ptr = scratch_dev[dev].load(std::memory_order_acquire);
    if (!ptr) {
        const hipError_t e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
        LFM2Q_REQUIRE(e == hipSuccess && ptr, LFM2Q_ERR_DEVICE,
                      "gemv_chain_noalloc: the scratch array's address on device %d: %s", dev, hipGetErrorString(e));
        scratch_dev[dev].store(ptr, std::memory_order_release);  // a racing first call stores the same address
    }
    *out = ptr;
    return LFM2Q_OK;
}

// zeroes n words (a kernel, not hipMemsetAsync, so that a captured graph replays it correctly)
__global__ __launch_bounds__(256) void clear_words_kernel(uint32_t *__restrict__ p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

}  // namespace
}  // namespace lfm2q

extern "C" size_t lfm2q_gemv_chain_workspace_bytes(void) { return (size_t)WS_WORDS * 4u; }

extern "C" int lfm2q_gemv_chain(const lfm2q_gemv_op *ops, const lfm2q_gemv_op *ops_dev, int n_ops, void *workspace,
                                size_t workspace_bytes, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(ops && ops_dev && workspace, LFM2Q_ERR_ARG, "gemv_chain: null pointer");
    LFM2Q_REQUIRE(n_ops >= 1 && n_ops <= MAX_OPS, LFM2Q_ERR_SHAPE, "gemv_chain: 1 to %d ops (got %d)", MAX_OPS, n_ops);
    LFM2Q_REQUIRE(workspace_bytes >= lfm2q_gemv_chain_workspace_bytes(), LFM2Q_ERR_SHAPE,
                  "gemv_chain: the workspace needs %zu bytes (got %zu)", lfm2q_gemv_chain_workspace_bytes(),
                  workspace_bytes);
    LFM2Q_REQUIRE(((uintptr_t)workspace & 255) == 0 && aligned16(ops_dev), LFM2Q_ERR_ALIGN,
                  "gemv_chain: the workspace must be 256-byte and the device op table 16-byte aligned");
    int G = 0;
    if (int st = check_chain("gemv_chain", ops, n_ops, G)) return st;
    return launch_chain("gemv_chain", ops_dev, n_ops, G, reinterpret_cast<uint32_t *>(workspace), nullptr,
                        (hipStream_t)stream);
}

extern "C" int lfm2q_gemv_chain_noalloc(const lfm2q_gemv_op *ops, const lfm2q_gemv_op *ops_dev, int n_ops,
                                        uint32_t *status, lfm2q_stream_t stream) {
    LFM2Q_REQUIRE(ops && ops_dev, LFM2Q_ERR_ARG, "gemv_chain_noalloc: null pointer");
    LFM2Q_REQUIRE(n_ops >= 1 && n_ops <= MAX_OPS, LFM2Q_ERR_SHAPE,
                  "gemv_chain_noalloc: 1 to %d ops (got %d): the chain's op table holds at most %d", MAX_OPS, n_ops,
                  MAX_OPS);
    LFM2Q_REQUIRE(aligned16(ops_dev) && ((uintptr_t)status & 3) == 0, LFM2Q_ERR_ALIGN,
                  "gemv_chain_noalloc: the device op table must be 16-byte and status 4-byte aligned");
    int G = 0;
    if (int st = check_chain("gemv_chain_noalloc", ops, n_ops, G)) return st;
    uint32_t *ws = nullptr;
    if (int st = scratch_of_current_device(&ws)) return st;
    // the previous call on this GPU left its flags, launch counter and error word: start from zeros
    clear_words_kernel<<<8, 256, 0, (hipStream_t)stream>>>(ws, WS_WORDS);
    if (int st = launch_status("gemv_chain_noalloc")) return st;
    return launch_chain("gemv_chain_noalloc", ops_dev, n_ops, G, ws, status, (hipStream_t)stream);
}
