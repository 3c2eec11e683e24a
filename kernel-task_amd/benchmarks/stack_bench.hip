// Persistent multi-layer stack of tensor-ring layers: L layers in one launch, alternating
// 1920->2880 and 2880->1920 (rank STACK_RANK, fp16), a grid-wide barrier between layers.
// Built by kernel-task_amd/benchmarks/stack_bench.py; prints one JSON object per (variant, L).
//
// Role of the reference's weight-stationary stack experiment (kernel_work/stack/tr_stack.cu:1-40,
// kernel-design/WEIGHT_STATIONARY.md:104-147): does one persistent kernel beat the same
// layers launched one by one? Own design on the MI355X kernel: every unit of a layer is one
// call of ring3_unit (the standalone kernel's body), each output owned by one workgroup, so
// there are no atomics on activations and the result is bitwise that of per-layer launches
// (checked here for every L). Two forms:
//   STACK_XCD 0  workgroups on every XCD; between layers a device-scope barrier (release:
//                write the L2 back; acquire: invalidate it), the only portable form
//   STACK_XCD 1  workgroups on one XCD (a grid of 8x the working workgroups, those dealt to
//                XCDs 1-7 exit at once): all of the stack shares one L2, so a barrier is an
//                atomic in that L2 plus an L1 invalidation; split into arrive (after a layer)
//                and wait (inside the next layer's first unit, once its core-slice loads are
//                in flight, which do not depend on the activations)
// Every barrier wait is bounded (it sets an error flag and gives up). The single stacks are
// cooperative launches, so the runtime refuses a grid whose workgroups could not all be
// resident; the side-by-side stacks (STACK_PAR) are plain launches, whose error flags are read
// after every run, the timed ones included, and refuse the figure when a barrier gave up.
// With STACK_DUMP=<dir> the program writes x, every layer's cores ([R][o][i][R], fp16) and
// every checked output (the stacks' and the per-layer launches') as raw fp16 files there, for
// a check against an independent restatement of each layer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "trk.h"
#include "trk_mfma_kernel.h"

using namespace trk;

#define CHECK(x)                                                                              \
    do {                                                                                      \
        auto e_ = (x);                                                                        \
        if (e_) {                                                                             \
            std::fprintf(stderr, "%s failed (%d) at line %d\n", #x, int(e_), __LINE__);       \
            std::exit(1);                                                                     \
        }                                                                                     \
    } while (0)

#ifndef STACK_RANK
#define STACK_RANK 8
#endif
#ifndef STACK_XCD
#define STACK_XCD 0
#endif

// layer shapes and their chain orders (the least padded MFMA work of each)
constexpr Shape kUp{TRK_DTYPE_F16, 2, 1, 0, 8, 12, 20, 12, 10, 24, STACK_RANK};
constexpr Shape kDown{TRK_DTYPE_F16, 2, 0, 1, 12, 10, 24, 8, 12, 20, STACK_RANK};
// tokens=1 tiles: every XCD, the tuned single-token tiles (4 waves); one XCD, tiles that own
// all second-core outputs (8 waves), so that 24 and 20 units fill most of its 32 CUs
#if STACK_XCD
constexpr KCfg CU = tile(kUp, 1, 1, 10, 12, 8, 4, 1, 0, 16, 8);
constexpr KCfg CD = tile(kDown, 1, 1, 8, 12, 10, 4, 1, 0, 16, 8);
#else
constexpr KCfg CU = tile(kUp, 1, 1, 2, 12, 8, 4, 1);
constexpr KCfg CD = tile(kDown, 1, 1, 2, 12, 10, 4, 1);
#endif
using GU = Geo<CU>;
using GD = Geo<CD>;
static_assert(GU::NT == GD::NT, "both layer tiles need the same workgroup size");
constexpr int NT = GU::NT;
constexpr int POOL = GU::LDS_ELEMS > GD::LDS_ELEMS ? GU::LDS_ELEMS : GD::LDS_ELEMS;
constexpr int NWG = GU::NBLK > GD::NBLK ? GU::NBLK : GD::NBLK;  // working workgroups
using E = typename Ops<CU.dt>::E;

struct Layer {
    const E *fk, *sk, *lk;
};

// device-scope barrier: every workgroup's stores written back from its L2 before it arrives,
// the L2 invalidated after the wait (the compiler's release/acquire at agent scope)
__device__ __forceinline__ void device_barrier(unsigned *counter, unsigned target, int *err,
                                               int spin) {
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        for (int n = 0; __hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) <
                        target;) {
            if (++n > spin) {
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// one-XCD barrier, arrive half: this workgroup's stores have reached the shared L2, then one
// atomic in that L2 (workgroup scope: no writeback)
__device__ __forceinline__ void xcd_arrive(unsigned *counter) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// one-XCD barrier, wait half. The counter is read with compare-and-swaps that never swap (it
// never holds 2^32 - 1): they execute in the L2 and return its value, while a plain load may
// be served a stale L1 line (and the compiler turns an atomic add of 0 into such a load).
// The layer's reads of its input activations then use device-scope loads (ring3_unit's
// COHERENT_X), which the CU's L1 does not serve, so they see the L2's current lines. (An L1
// invalidation at workgroup scope, `buffer_inv sc0`, was not enough: outside threadgroup-split
// mode a workgroup's waves share one L1, so that scope need not touch it, and stale lines of
// an activation buffer from two layers back were read, 1 run in ~8 giving wrong outputs. The
// device-scope invalidation, `buffer_inv sc1`, made each barrier cost 11.7 µs.)
__device__ __forceinline__ void xcd_wait(unsigned *counter, unsigned target, int *err, int spin) {
    if (threadIdx.x == 0) {
        for (int n = 0;;) {
            unsigned v = 0xffffffffu;
            __hip_atomic_compare_exchange_strong(counter, &v, 0xffffffffu, __ATOMIC_RELAXED,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (v >= target) break;
            if (++n > spin) {
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// This workgroup's units of one layer. A nonzero target means the previous layer's barrier is
// still open: with PREFETCH the first unit waits inside ring3_unit once its core-slice loads
// are in flight; without, before it starts; a workgroup without a unit waits at the end.
template <KCfg C, bool PREFETCH>
__device__ __forceinline__ void run_layer(const Layer &lay, const E *in, E *out, int T, int wg,
                                          E *pool, unsigned *counter, unsigned target, int *err,
                                          int spin) {
    using G = Geo<C>;
    const int units = G::NBLK * ((T + G::TT - 1) / G::TT);
    bool pending = target != 0;
    for (int u = wg; u < units; u += NWG) {
        auto wait = [&]() {
            if (pending) xcd_wait(counter, target, err, spin);
            pending = false;
        };
        // the one-XCD form reads the activations with device-scope loads (see xcd_wait); the
        // device-scope barrier of the other form invalidates the CU's L1 itself
        constexpr bool COHERENT = STACK_XCD != 0;
        if constexpr (PREFETCH) {
            ring3_unit<C, false, decltype((wait)), false, COHERENT>(
                in, lay.fk, lay.sk, lay.lk, out, T, 0, nullptr, u % G::NBLK, u / G::NBLK,
                pool + G::oFs, pool + G::oSs, pool + G::oLs, pool + G::oXs, pool + G::oUb,
                pool + G::oVb, wait);
        } else {
            wait();
            ring3_unit<C, false, NoHook, false, COHERENT>(
                in, lay.fk, lay.sk, lay.lk, out, T, 0, nullptr, u % G::NBLK, u / G::NBLK,
                pool + G::oFs, pool + G::oSs, pool + G::oLs, pool + G::oXs, pool + G::oUb,
                pool + G::oVb);
        }
        __syncthreads();  // the next unit reuses the LDS
    }
    if (pending) xcd_wait(counter, target, err, spin);
}

// WORK false: the barriers alone. Layer l reads x (l = 0) or act[(l-1) & 1] and writes y
// (l = L-1) or act[l & 1]. The counter only grows: launch k waits for base + l * NWG.
template <bool WORK, bool PREFETCH>
__global__ void __launch_bounds__(NT)
    stack_kernel(const E *x, E *act0, E *act1, E *y, const Layer *layers, int L, int T,
                 unsigned *counter, unsigned base, int *err, int spin, unsigned *xcc, int xcd) {
    __shared__ __attribute__((aligned(16))) E pool[POOL];
    int wg = blockIdx.x;
    if constexpr (STACK_XCD) {
        // the XCD this workgroup runs on (hardware register XCC_ID, bits 3:0): the host
        // checks that every working workgroup ran on one XCD, which the L2 barrier assumes
        unsigned id;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(id));
        id &= 0xfu;
        // xcd < 0: the workgroups of residue 0 modulo 8 work (one launch at a time, dealt from
        // XCD 0). xcd >= 0: those running on XCD `xcd` work, for launches side by side whose
        // dealing starts at different XCDs; round-robin dealing puts one residue class
        // modulo 8 on each XCD, so wg / 8 still numbers them 0..NWG-1
        if (xcd < 0 ? wg % 8 != 0 : int(id) != xcd) return;
        wg /= 8;
        if (threadIdx.x == 0) xcc[wg] = id;
    }
    for (int l = 0; l < L; ++l) {
        const E *in = l == 0 ? x : ((l - 1) & 1 ? act1 : act0);
        E *out = l == L - 1 ? y : (l & 1 ? act1 : act0);
        if constexpr (STACK_XCD) {
            const unsigned target = l > 0 ? base + unsigned(l) * NWG : 0u;
            if constexpr (WORK) {
                if (l % 2 == 0)
                    run_layer<CU, PREFETCH>(layers[l], in, out, T, wg, pool, counter, target, err, spin);
                else
                    run_layer<CD, PREFETCH>(layers[l], in, out, T, wg, pool, counter, target, err, spin);
            } else if (target) {
                xcd_wait(counter, target, err, spin);
            }
            if (l + 1 < L) xcd_arrive(counter);
        } else {
            if constexpr (WORK) {
                if (l % 2 == 0)
                    run_layer<CU, false>(layers[l], in, out, T, wg, pool, counter, 0u, err, spin);
                else
                    run_layer<CD, false>(layers[l], in, out, T, wg, pool, counter, 0u, err, spin);
            }
            if (l + 1 < L) device_barrier(counter, base + unsigned(l + 1) * NWG, err, spin);
        }
    }
}

int main(int argc, char **argv) {
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    const int T = argc > 1 ? std::atoi(argv[1]) : 1;
    std::vector<int> Ls;
    for (int a = 2; a < argc; ++a) Ls.push_back(std::atoi(argv[a]));
    if (Ls.empty()) Ls = {8, 32, 128};
    if (T < 1 || T > 64 || *std::min_element(Ls.begin(), Ls.end()) < 1) {
        std::fprintf(stderr, "usage: stack_bench T(1..64) L [L ...]\n");
        return 2;
    }
    const int Lmax = *std::max_element(Ls.begin(), Ls.end());
    const int R = STACK_RANK;
    const int m_up[3] = {8, 12, 20}, m_down[3] = {12, 10, 24};
    trk_plan *pu, *pd;
    CHECK(trk_plan_create(m_up, m_down, R, TRK_DTYPE_F16, &pu));
    CHECK(trk_plan_create(m_down, m_up, R, TRK_DTYPE_F16, &pd));
    const int ou[3] = {CU.F, CU.S, CU.L}, od[3] = {CD.F, CD.S, CD.L};
    Plan *PU = reinterpret_cast<Plan *>(pu), *PD = reinterpret_cast<Plan *>(pd);
    const int cu = plan_chain(PU, ou, s_group(CU), l_group(CU), s_frag(CU));
    const int cd = plan_chain(PD, od, s_group(CD), l_group(CD), s_frag(CD));
    if (cu < 0 || cd < 0) {
        std::fprintf(stderr, "no packed chain for the stack's tiles\n");
        return 1;
    }
    const char *dump = std::getenv("STACK_DUMP");
    auto write_file = [&](const std::string &name, const void *data, size_t bytes) {
        if (!dump) return;
        const std::string path = std::string(dump) + "/" + name;
        FILE *f = std::fopen(path.c_str(), "wb");
        if (!f || std::fwrite(data, 1, bytes, f) != bytes) {
            std::fprintf(stderr, "cannot write %s\n", path.c_str());
            std::exit(1);
        }
        std::fclose(f);
    };
    std::mt19937 rng(7);
    std::normal_distribution<float> nd(0.f, 1.f);
    // distinct cores per layer, per-core sigma (make_cores) so activations stay O(1)
    std::vector<void *> owned;
    auto make_layer = [&](trk_plan *p, const int *in, const int *out, int chain, int l) {
        const double sig = std::pow(double(in[0] * in[1] * in[2]) * R * R * R, -1.0 / 6.0);
        void *g[3];
        for (int k = 0; k < 3; ++k) {
            const size_t n = size_t(R) * out[k] * in[k] * R;
            std::vector<E> h(n);
            for (auto &v : h) v = E(float(nd(rng) * sig));
            write_file("core_l" + std::to_string(l) + "_k" + std::to_string(k) + ".bin", h.data(),
                       n * sizeof(E));
            CHECK(hipMalloc(&g[k], n * sizeof(E)));
            CHECK(hipMemcpy(g[k], h.data(), n * sizeof(E), hipMemcpyHostToDevice));
        }
        char *packed;
        CHECK(hipMalloc(&packed, trk_plan_packed_bytes(p)));
        owned.push_back(packed);
        CHECK(trk_pack(p, g[0], g[1], g[2], packed, nullptr));
        CHECK(hipDeviceSynchronize());
        for (int k = 0; k < 3; ++k) CHECK(hipFree(g[k]));
        const Chain &c = reinterpret_cast<Plan *>(p)->chains[chain];
        return Layer{reinterpret_cast<const E *>(packed + c.offF),
                     reinterpret_cast<const E *>(packed + c.offS),
                     reinterpret_cast<const E *>(packed + c.offL)};
    };
    std::vector<Layer> layers;
    for (int l = 0; l < Lmax; ++l)
        layers.push_back(l % 2 == 0 ? make_layer(pu, m_up, m_down, cu, l)
                                    : make_layer(pd, m_down, m_up, cd, l));
    Layer *dlayers;
    CHECK(hipMalloc(&dlayers, sizeof(Layer) * Lmax));
    CHECK(hipMemcpy(dlayers, layers.data(), sizeof(Layer) * Lmax, hipMemcpyHostToDevice));
    constexpr int MAXF = 2880;  // widest activation row
    std::vector<E> hx(size_t(T) * 1920);
    for (auto &v : hx) v = E(nd(rng));
    write_file("x.bin", hx.data(), hx.size() * sizeof(E));
    E *x, *a0, *a1, *y, *yr, *b0, *b1;
    CHECK(hipMalloc(&x, hx.size() * sizeof(E)));
    CHECK(hipMemcpy(x, hx.data(), hx.size() * sizeof(E), hipMemcpyHostToDevice));
    for (E **p : {&a0, &a1, &y, &yr, &b0, &b1}) CHECK(hipMalloc(p, size_t(T) * MAXF * sizeof(E)));
    unsigned *counter, *xcc;
    int *err;
    CHECK(hipMalloc(&counter, sizeof(unsigned)));
    CHECK(hipMalloc(&xcc, sizeof(unsigned) * NWG));
    CHECK(hipMalloc(&err, sizeof(int)));
    CHECK(hipMemset(counter, 0, sizeof(unsigned)));
    CHECK(hipMemset(err, 0, sizeof(int)));
    const int grid = STACK_XCD ? 8 * NWG : NWG;
    const int spin = 1 << 14;  // polls of ~27 ns: ~0.4 ms before a barrier gives up
    unsigned base = 0;

    auto per_layer = [&](int L, hipStream_t s) {  // the same tiles, one standalone launch each
        for (int l = 0; l < L; ++l) {
            const E *in = l == 0 ? x : ((l - 1) & 1 ? b1 : b0);
            E *out = l == L - 1 ? yr : (l & 1 ? b1 : b0);
            if (l % 2 == 0)
                hipLaunchKernelGGL((ring3_mfma_kernel<CU, false>), dim3(GU::NBLK, (T + GU::TT - 1) / GU::TT),
                                   dim3(NT), 0, s, in, layers[l].fk, layers[l].sk, layers[l].lk,
                                   (void *)out, T, 0, (const void *)nullptr);
            else
                hipLaunchKernelGGL((ring3_mfma_kernel<CD, false>), dim3(GD::NBLK, (T + GD::TT - 1) / GD::TT),
                                   dim3(NT), 0, s, in, layers[l].fk, layers[l].sk, layers[l].lk,
                                   (void *)out, T, 0, (const void *)nullptr);
        }
    };
    auto stack = [&](int L, bool work, bool prefetch) {
        int Ti = T, Li = L, spini = spin, xcd0 = -1;
        void *args[] = {&x, &a0, &a1, &y, &dlayers, &Li, &Ti, &counter, &base, &err, &spini, &xcc,
                        &xcd0};
        const void *fn = work ? (prefetch ? (const void *)stack_kernel<true, true>
                                          : (const void *)stack_kernel<true, false>)
                              : (const void *)stack_kernel<false, false>;
        CHECK(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, 0, nullptr));
        base += unsigned(L - 1) * NWG;
    };
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    auto time_us = [&](auto &&fn, int reps) {  // median of 5 blocks of back-to-back calls
        for (int i = 0; i < 3; ++i) fn();
        CHECK(hipDeviceSynchronize());
        std::vector<float> t;
        for (int r = 0; r < 5; ++r) {
            CHECK(hipEventRecord(e0, nullptr));
            for (int i = 0; i < reps; ++i) fn();
            CHECK(hipEventRecord(e1, nullptr));
            CHECK(hipEventSynchronize(e1));
            float ms;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            t.push_back(ms * 1000.f / reps);
        }
        std::sort(t.begin(), t.end());
        return t[2];
    };
#if STACK_XCD
    if (const char *par = std::getenv("STACK_PAR")) {
        // P independent stacks at once, stack k on XCD k (P sequences through one model, each
        // confined to its own XCD's L2), against one stack alone and against the same tiles
        // launched per layer for a batch of the P tokens. Plain launches: a stack whose
        // workgroups were not all resident at once would end its barriers at the spin bound
        // and report it.
        const int P = std::atoi(par);
        if (P < 1 || P > 8 || T != 1) {
            std::fprintf(stderr, "STACK_PAR wants 1..8 stacks at T=1\n");
            return 2;
        }
        std::vector<hipStream_t> st(P);
        std::vector<hipEvent_t> ek(P);
        std::vector<E *> pa0(P), pa1(P), py(P);
        std::vector<unsigned *> pcnt(P), pxcc(P);
        std::vector<int *> perr(P);
        std::vector<unsigned> pbase(P, 0u);
        for (int k = 0; k < P; ++k) {
            CHECK(hipStreamCreate(&st[k]));
            CHECK(hipEventCreateWithFlags(&ek[k], hipEventDisableTiming));
            for (E **q : {&pa0[k], &pa1[k], &py[k]}) CHECK(hipMalloc(q, MAXF * sizeof(E)));
            CHECK(hipMalloc(&pcnt[k], sizeof(unsigned)));
            CHECK(hipMalloc(&perr[k], sizeof(int)));
            CHECK(hipMalloc(&pxcc[k], sizeof(unsigned) * NWG));
            CHECK(hipMemset(pcnt[k], 0, sizeof(unsigned)));
            CHECK(hipMemset(perr[k], 0, sizeof(int)));
        }
        E *xb, *c0, *c1, *yb;  // the batch: x's row P times
        CHECK(hipMalloc(&xb, size_t(P) * 1920 * sizeof(E)));
        for (int k = 0; k < P; ++k)
            CHECK(hipMemcpy(xb + size_t(k) * 1920, x, 1920 * sizeof(E), hipMemcpyDeviceToDevice));
        for (E **q : {&c0, &c1, &yb}) CHECK(hipMalloc(q, size_t(P) * MAXF * sizeof(E)));
        hipEvent_t ej;
        CHECK(hipEventCreateWithFlags(&ej, hipEventDisableTiming));
        auto launch_k = [&](int k, int L, hipStream_t s) {
            int Ti = 1, Li = L, spini = spin, xk = k;
            void *args[] = {&x, &pa0[k], &pa1[k], &py[k], &dlayers, &Li, &Ti, &pcnt[k], &pbase[k],
                            &perr[k], &spini, &pxcc[k], &xk};
            CHECK(hipLaunchKernel((const void *)stack_kernel<true, true>, dim3(8 * NWG), dim3(NT),
                                  args, 0, s));
            pbase[k] += unsigned(L - 1) * NWG;
        };
        auto all = [&](int L) {  // the P stacks side by side, joined on the null stream
            CHECK(hipEventRecord(ej, nullptr));
            for (int k = 0; k < P; ++k) {
                CHECK(hipStreamWaitEvent(st[k], ej, 0));
                launch_k(k, L, st[k]);
                CHECK(hipEventRecord(ek[k], st[k]));
            }
            for (int k = 0; k < P; ++k) CHECK(hipStreamWaitEvent(nullptr, ek[k], 0));
        };
        auto batch = [&](int L) {  // the same tiles per layer, P tokens
            for (int l = 0; l < L; ++l) {
                const E *in = l == 0 ? xb : ((l - 1) & 1 ? c1 : c0);
                E *out = l == L - 1 ? yb : (l & 1 ? c1 : c0);
                if (l % 2 == 0)
                    hipLaunchKernelGGL((ring3_mfma_kernel<CU, false>), dim3(GU::NBLK, (P + GU::TT - 1) / GU::TT),
                                       dim3(NT), 0, nullptr, in, layers[l].fk, layers[l].sk,
                                       layers[l].lk, (void *)out, P, 0, (const void *)nullptr);
                else
                    hipLaunchKernelGGL((ring3_mfma_kernel<CD, false>), dim3(GD::NBLK, (P + GD::TT - 1) / GD::TT),
                                       dim3(NT), 0, nullptr, in, layers[l].fk, layers[l].sk,
                                       layers[l].lk, (void *)out, P, 0, (const void *)nullptr);
            }
        };
        for (int L : Ls) {
            const int reps = std::max(2, 500 / L);
            for (int k = 0; k < P; ++k) {
                CHECK(hipMemset(py[k], 0xff, MAXF * sizeof(E)));
                CHECK(hipMemset(pxcc[k], 0xff, sizeof(unsigned) * NWG));
            }
            all(L);
            per_layer(L, nullptr);
            CHECK(hipDeviceSynchronize());
            const int outn = L % 2 == 1 ? 2880 : 1920;
            std::vector<E> h2(outn), h1(outn);
            CHECK(hipMemcpy(h2.data(), yr, outn * sizeof(E), hipMemcpyDeviceToHost));
            write_file("yref_L" + std::to_string(L) + ".bin", h2.data(), outn * sizeof(E));
            size_t diff = 0, missing = 0;
            int timeouts = 0;
            std::string ids;
            for (int k = 0; k < P; ++k) {
                CHECK(hipMemcpy(h1.data(), py[k], outn * sizeof(E), hipMemcpyDeviceToHost));
                write_file("ypar" + std::to_string(k) + "_L" + std::to_string(L) + ".bin",
                           h1.data(), outn * sizeof(E));
                for (int i = 0; i < outn; ++i) diff += std::memcmp(&h1[i], &h2[i], sizeof(E)) != 0;
                int herr = 0;
                CHECK(hipMemcpy(&herr, perr[k], sizeof(int), hipMemcpyDeviceToHost));
                timeouts += herr;
                std::vector<unsigned> hids(NWG);
                CHECK(hipMemcpy(hids.data(), pxcc[k], sizeof(unsigned) * NWG, hipMemcpyDeviceToHost));
                // a unit no workgroup took keeps the fill: the dealing was not one residue class
                // per XCD (then some other unit ran twice)
                missing += std::count(hids.begin(), hids.end(), 0xffffffffu);
                hids.erase(std::remove(hids.begin(), hids.end(), 0xffffffffu), hids.end());
                std::sort(hids.begin(), hids.end());
                hids.erase(std::unique(hids.begin(), hids.end()), hids.end());
                ids += k ? ", [" : "[";
                for (size_t j = 0; j < hids.size(); ++j)
                    ids += (j ? ", " : "") + std::to_string(int(hids[j]));
                ids += "]";
            }
            if (timeouts) {
                std::printf("{\"form\": \"one_xcd_parallel\", \"stacks\": %d, \"layers\": %d, "
                            "\"error\": \"a barrier reached its spin bound\", \"units_missing\": %zu, "
                            "\"xcd_ids\": [%s]}\n", P, L, missing, ids.c_str());
                continue;
            }
            const float t_all = time_us([&] { all(L); }, reps);
            const float t_one = time_us([&] { launch_k(0, L, nullptr); }, reps);
            const float t_batch = time_us([&] { batch(L); }, reps);
            // the timed runs' barriers too: a stack that gave up waiting ran a layer early
            int timed_timeouts = 0;
            for (int k = 0; k < P; ++k) {
                int herr = 0;
                CHECK(hipMemcpy(&herr, perr[k], sizeof(int), hipMemcpyDeviceToHost));
                timed_timeouts += herr;
            }
            if (timed_timeouts) {
                std::printf("{\"form\": \"one_xcd_parallel\", \"stacks\": %d, \"layers\": %d, "
                            "\"error\": \"a barrier reached its spin bound in a timed run\", "
                            "\"xcd_ids\": [%s]}\n", P, L, ids.c_str());
                continue;
            }
            std::printf("{\"form\": \"one_xcd_parallel\", \"stacks\": %d, \"rank\": %d, \"layers\": %d, "
                        "\"parallel_us\": %.3f, \"one_stack_us\": %.3f, \"batched_per_layer_us\": %.3f, "
                        "\"outputs_differing\": %zu, \"outputs\": %d, \"units_missing\": %zu, "
                        "\"xcd_ids\": [%s]}\n",
                        P, R, L, t_all, t_one, t_batch, diff, outn * P, missing, ids.c_str());
        }
        return 0;
    }
#endif
    const bool prefetch_modes[2] = {false, true};
    for (int L : Ls) {
        const int reps = std::max(2, 2000 / L);
        hipStream_t cs;
        CHECK(hipStreamCreate(&cs));
        hipGraph_t g;
        hipGraphExec_t ge;
        CHECK(hipStreamBeginCapture(cs, hipStreamCaptureModeGlobal));
        per_layer(L, cs);
        CHECK(hipStreamEndCapture(cs, &g));
        CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        const float t_eager = time_us([&] { per_layer(L, nullptr); }, reps);
        const float t_graph = time_us([&] { CHECK(hipGraphLaunch(ge, nullptr)); }, reps);
        const float t_bar = time_us([&] { stack(L, false, false); }, reps);
        for (int m = 0; m < (STACK_XCD ? 2 : 1); ++m) {
            const bool pf = prefetch_modes[m];
            // correctness: bitwise against the per-layer launches of the same tiles
            CHECK(hipMemset(y, 0xff, size_t(T) * MAXF * sizeof(E)));
            CHECK(hipMemset(xcc, 0xff, sizeof(unsigned) * NWG));
            stack(L, true, pf);
            per_layer(L, nullptr);
            CHECK(hipDeviceSynchronize());
            int herr = 0;
            CHECK(hipMemcpy(&herr, err, sizeof(int), hipMemcpyDeviceToHost));
            if (herr) {
                std::printf("{\"error\": \"a barrier reached its spin bound\", \"L\": %d}\n", L);
                return 3;
            }
            std::vector<unsigned> hids(NWG);
            CHECK(hipMemcpy(hids.data(), xcc, sizeof(unsigned) * NWG, hipMemcpyDeviceToHost));
            std::sort(hids.begin(), hids.end());
            hids.erase(std::unique(hids.begin(), hids.end()), hids.end());
            std::string ids;
            for (unsigned v : hids) ids += (ids.empty() ? "" : ", ") + std::to_string(int(v));
            const int outn = (L % 2 == 1 ? 2880 : 1920) * T;
            std::vector<E> h1(outn), h2(outn);
            CHECK(hipMemcpy(h1.data(), y, outn * sizeof(E), hipMemcpyDeviceToHost));
            CHECK(hipMemcpy(h2.data(), yr, outn * sizeof(E), hipMemcpyDeviceToHost));
            const std::string tag = std::string(STACK_XCD ? "xcd" : "all") + "_T" +
                                    std::to_string(T) + "_L" + std::to_string(L);
            write_file("y_" + tag + (pf ? "_pf1.bin" : "_pf0.bin"), h1.data(), outn * sizeof(E));
            write_file("yref_" + tag + ".bin", h2.data(), outn * sizeof(E));
            // a differing output still holding the fill pattern was never written
            size_t diff = 0, unwritten = 0;
            int first = -1;
            const unsigned short fill = 0xffffu;
            for (int i = 0; i < outn; ++i) {
                if (std::memcmp(&h1[i], &h2[i], sizeof(E)) == 0) continue;
                ++diff;
                unwritten += std::memcmp(&h1[i], &fill, sizeof(E)) == 0;
                if (first < 0) first = i;
            }
            const float t_stack = time_us([&] { stack(L, true, pf); }, reps);
            CHECK(hipMemcpy(&herr, err, sizeof(int), hipMemcpyDeviceToHost));
            std::printf("{\"form\": \"%s\", \"prefetch\": %s, \"rank\": %d, \"tokens\": %d, \"layers\": %d, "
                        "\"workgroups\": %d, \"stack_us\": %.3f, \"barriers_only_us\": %.3f, "
                        "\"per_layer_eager_us\": %.3f, \"per_layer_graph_us\": %.3f, "
                        "\"outputs_differing\": %zu, \"differing_unwritten\": %zu, "
                        "\"first_differing\": %d, \"outputs\": %d, \"barrier_timeouts\": %d, "
                        "\"xcd_ids\": [%s]}\n",
                        STACK_XCD ? "one_xcd" : "all_xcds", pf ? "true" : "false", R, T, L, NWG,
                        t_stack, t_bar, t_eager, t_graph, diff, unwritten, first, outn, herr,
                        STACK_XCD ? ids.c_str() : "");
        }
        CHECK(hipGraphExecDestroy(ge));
        CHECK(hipGraphDestroy(g));
        CHECK(hipStreamDestroy(cs));
    }
    for (void *p : owned) CHECK(hipFree(p));
    CHECK(hipFree(xcc));
    trk_plan_destroy(pu);
    trk_plan_destroy(pd);
    return 0;
}
