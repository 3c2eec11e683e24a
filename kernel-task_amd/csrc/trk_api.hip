// C ABI entry points of libtrk: plans, packing, forward, floors.
//
// A plan fixes one operator shape and dtype, the contraction orders its kernels use (each
// with a section of the packed-core buffer) and a table of kernel variants with the token
// counts each one serves. Host-only logic: nothing here calls HIP except trk_pack,
// trk_forward* and trk_empty_launch.
#include <dlfcn.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

#include "trk_internal.h"

namespace trk {

namespace {
thread_local char g_error[512] = "";

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
int round_up(int v, int m) { return (v + m - 1) / m * m; }

// multiply-adds x 2 per token of chain c at ring rank `rank` (the plan's kernel rank for the
// work its kernels do, its core rank for the algorithmic work)
double chain_flops_per_token(const Plan &p, const Chain &c, int rank) {
    const double R = rank;
    const double s1 = double(p.in_features) * c.oF * R * R;
    const double s2 = double(c.nS) * c.nL * c.oF * c.oS * R * R * R;
    const double s3 = double(c.nL) * p.out_features * R * R;
    return 2.0 * (s1 + s2 + s3);
}

const Plan *as_plan(const trk_plan *plan) { return reinterpret_cast<const Plan *>(plan); }
Plan *as_plan(trk_plan *plan) { return reinterpret_cast<Plan *>(plan); }

void grid_of(const Plan &p, const Variant &v, int tokens, int grid[3]) {
    const Chain &c = p.chains[v.chain];
    if (v.kind == TRK_KERNEL_GENERIC) {
        grid[0] = c.oF * ((c.oS + v.tile[2] - 1) / v.tile[2]);
        grid[1] = std::max(1, std::min(tokens, 65535));
        grid[2] = 1;
    } else {
        const int TT = v.tile[0], FC = v.tile[1], SC = v.tile[2], LC = v.tile[3];
        grid[0] = ((c.oF + FC - 1) / FC) * ((c.oS + SC - 1) / SC) * ((c.oL + LC - 1) / LC) *
                  (v.xcd_local ? 8 / v.xcd_local : 1);
        grid[1] = std::max(1, (tokens + TT - 1) / TT);
        grid[2] = 1;
    }
}
}  // namespace

// Index of the chain with this order and these K-order groups in the plan, adding it (and
// the packed sections it does not share with an earlier chain of the same order).
int plan_chain(Plan *p, const int order[3], int sg, int lg, int sfrag) {
    auto same_order = [&](const Chain &c) { return std::equal(order, order + 3, c.order); };
    for (int i = 0; i < p->nchains; ++i) {
        const Chain &o = p->chains[i];
        if (same_order(o) && o.sg == sg && o.lg == lg && o.sfrag == sfrag) return i;
    }
    if (p->nchains == kMaxChains) return -1;
    Chain &c = p->chains[p->nchains];
    describe_chain(p->in_modes, p->out_modes, p->rank, order, &c);
    c.sg = sg;
    c.lg = lg;
    c.sfrag = sfrag;
    c.ownF = c.ownS = c.ownL = 1;
    // sections whose layout an earlier chain of this order already has are shared
    for (int i = 0; i < p->nchains; ++i) {
        const Chain &o = p->chains[i];
        if (!same_order(o)) continue;
        if (c.ownF) { c.offF = o.offF; c.ownF = 0; }
        if (c.ownS && o.sg == sg && o.sfrag == sfrag) { c.offS = o.offS; c.ownS = 0; }
        if (c.ownL && o.lg == lg) { c.offL = o.offL; c.ownL = 0; }
    }
    const size_t e = size_t(p->elem);
    auto take = [&](size_t elems) {
        const size_t off = p->packed_bytes;
        p->packed_bytes = align256(off + e * elems);
        return off;
    };
    if (c.ownF) c.offF = take(size_t(c.oF) * c.R * c.R * c.KF);
    if (c.ownS) c.offS = take(size_t(sfrag ? round_up(c.oS * c.R, 32) : c.oS * c.R) * c.K2);
    if (c.ownL) c.offL = take(size_t(c.nL) * c.oL * c.R * c.R);
    return p->nchains++;
}

int set_error(int status, const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
    return status;
}

int check_hip(hipError_t err, const char *what) {
    if (err == hipSuccess) return TRK_OK;
    return set_error(TRK_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

void describe_chain(const int in_modes[3], const int out_modes[3], int rank, const int order[3],
                    Chain *c) {
    const int F = order[0], S = order[1], L = order[2];
    std::copy(order, order + 3, c->order);
    c->forward = ((S - F + 3) % 3) == 1;
    c->nF = in_modes[F];
    c->nS = in_modes[S];
    c->nL = in_modes[L];
    c->oF = out_modes[F];
    c->oS = out_modes[S];
    c->oL = out_modes[L];
    c->R = rank;
    c->KF = round_up(c->nF, 16);
    c->K2 = round_up(c->nS * rank, 16);
    const int sx[3] = {in_modes[1] * in_modes[2], in_modes[2], 1};
    const int sy[3] = {out_modes[1] * out_modes[2], out_modes[2], 1};
    c->sxF = sx[F];
    c->sxS = sx[S];
    c->sxL = sx[L];
    c->syF = sy[F];
    c->syS = sy[S];
    c->syL = sy[L];
    c->offF = c->offS = c->offL = 0;
}

}  // namespace trk

using namespace trk;

extern "C" {

int trk_abi_version(void) { return TRK_ABI_VERSION; }

const char *trk_last_error(void) { return g_error; }

int trk_plan_create(const int in_modes[3], const int out_modes[3], int rank, int dtype,
                    trk_plan **out) {
    return trk_plan_create_padded(in_modes, out_modes, rank, rank, dtype, out);
}

int trk_plan_create_padded(const int in_modes[3], const int out_modes[3], int core_rank,
                           int rank, int dtype, trk_plan **out) {
    g_error[0] = '\0';
    if (!out || !in_modes || !out_modes)
        return set_error(TRK_ERR_INVALID, "trk_plan_create: null argument");
    *out = nullptr;
    for (int m = 0; m < 3; ++m)
        if (in_modes[m] <= 0 || out_modes[m] <= 0)
            return set_error(TRK_ERR_INVALID, "trk_plan_create: modes must be positive");
    if (core_rank <= 0) return set_error(TRK_ERR_INVALID, "trk_plan_create: rank must be positive");
    if (rank < core_rank)
        return set_error(TRK_ERR_INVALID, "trk_plan_create: kernel rank %d below the cores' rank %d",
                         rank, core_rank);
    if (dtype != TRK_DTYPE_F16 && dtype != TRK_DTYPE_BF16 && dtype != TRK_DTYPE_F32)
        return set_error(TRK_ERR_INVALID, "trk_plan_create: unknown dtype %d", dtype);
    const long long in_f = 1LL * in_modes[0] * in_modes[1] * in_modes[2];
    const long long out_f = 1LL * out_modes[0] * out_modes[1] * out_modes[2];
    if (in_f > (1LL << 28) || out_f > (1LL << 28) || rank > 64)
        return set_error(TRK_ERR_UNSUPPORTED, "trk_plan_create: shape too large");

    Plan *p = new (std::nothrow) Plan();
    if (!p) return set_error(TRK_ERR_NOMEM, "trk_plan_create: out of host memory");
    std::copy(in_modes, in_modes + 3, p->in_modes);
    std::copy(out_modes, out_modes + 3, p->out_modes);
    p->rank = rank;
    p->core_rank = core_rank;
    p->dtype = dtype;
    p->elem = dtype == TRK_DTYPE_F32 ? 4 : 2;
    p->in_features = int(in_f);
    p->out_features = int(out_f);

    // The generic kernel runs the order with the fewest flops (ties: the reference's order,
    // then the listed order).
    static const int kOrders[6][3] = {{0, 1, 2}, {1, 2, 0}, {2, 0, 1},
                                      {0, 2, 1}, {1, 0, 2}, {2, 1, 0}};
    int best = 0;
    double best_flops = 0.0;
    for (int o = 0; o < 6; ++o) {
        Chain c;
        describe_chain(in_modes, out_modes, rank, kOrders[o], &c);
        const double fl = chain_flops_per_token(*p, c, rank);
        if (o == 0 || fl < best_flops * (1.0 - 1e-9)) {
            best = o;
            best_flops = fl;
        }
    }
    // Variant 0: one workgroup per (token, first-core output) owns all second-core outputs;
    // it serves every token count no other variant claims. Variant 1, when the shape has
    // few first-core outputs: the second-core outputs are split over workgroups as well
    // (stage 1 recomputed per split, the rank^3 stage divided), for token counts too small
    // to fill the GPU with variant 0's workgroups.
    Variant &g = p->variants[0];
    // the K-order groups of the MFMA chains of the same order where the rank allows them
    // (sections shared), the natural orders otherwise
    const int kg = p->rank % 4 == 0 && p->rank != 8 ? 4 : p->rank;
    g.chain = plan_chain(p, kOrders[best], kg, kg, 0);
    const Chain &gc = p->chains[g.chain];
    int st = generic_configure(*p, g.chain, gc.oS, &g);
    if (st != TRK_OK) {
        delete p;
        return st;
    }
    g.t_min = 1;
    g.t_max = 1 << 30;
    p->nvariants = 1;
    constexpr int kFillGroups = 512;  // two workgroups per CU
    const int nsg = std::min(gc.oS, std::max(1, kFillGroups / gc.oF));
    const int sg = (gc.oS + nsg - 1) / nsg;
    if (sg < gc.oS) {
        Variant &spread = p->variants[1];
        if (generic_configure(*p, g.chain, sg, &spread) == TRK_OK) {
            spread.t_min = 1;
            // measured on MI355X: the split wins while variant 0 has at most ~64 workgroups
            spread.t_max = std::max(1, 64 / gc.oF);
            p->nvariants = 2;
        }
        g_error[0] = '\0';
    }
    mfma_register_generated(p);
    *out = reinterpret_cast<trk_plan *>(p);
    return TRK_OK;
}

int trk_plan_load_module(trk_plan *plan, const char *path, int *added) {
    if (added) *added = 0;
    if (!plan || !path) return set_error(TRK_ERR_INVALID, "trk_plan_load_module: null argument");
    // loaded once per process and never closed: the plan's variants point into the module
    void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!h) return set_error(TRK_ERR_INVALID, "trk_plan_load_module: %s", dlerror());
    auto abi = reinterpret_cast<int (*)()>(dlsym(h, kModuleAbi));
    auto size = reinterpret_cast<ModuleSizeFn>(dlsym(h, kModulePlanSize));
    auto reg = reinterpret_cast<ModuleRegisterFn>(dlsym(h, kModuleRegister));
    if (!abi || !size || !reg)
        return set_error(TRK_ERR_INVALID, "trk_plan_load_module: %s is not a variant module", path);
    if (abi() != TRK_ABI_VERSION || size() != sizeof(Plan))
        return set_error(TRK_ERR_INVALID,
                         "trk_plan_load_module: %s was built for ABI %d, plan size %zu (this "
                         "library: ABI %d, plan size %zu)", path, abi(), size(), TRK_ABI_VERSION,
                         sizeof(Plan));
    const int n = reg(as_plan(plan));
    if (added) *added = n;
    return TRK_OK;
}

void trk_plan_destroy(trk_plan *plan) { delete as_plan(plan); }

size_t trk_plan_packed_bytes(const trk_plan *plan) {
    return plan ? as_plan(plan)->packed_bytes : 0;
}

int trk_plan_variant_count(const trk_plan *plan) { return plan ? as_plan(plan)->nvariants : 0; }

int trk_plan_select(const trk_plan *plan, int tokens) {
    if (!plan) return -1;
    const Plan &p = *as_plan(plan);
    // later entries were registered for narrower token ranges and win over earlier ones
    for (int i = p.nvariants - 1; i > 0; --i)
        if (tokens >= p.variants[i].t_min && tokens <= p.variants[i].t_max && p.variants[i].t_min > 0)
            return i;
    return 0;
}

int trk_plan_describe(const trk_plan *plan, int variant, int tokens, trk_variant_info *info) {
    if (!plan || !info) return set_error(TRK_ERR_INVALID, "trk_plan_describe: null argument");
    const Plan &p = *as_plan(plan);
    if (tokens < 0) return set_error(TRK_ERR_INVALID, "trk_plan_describe: tokens < 0");
    if (variant < 0) variant = trk_plan_select(plan, tokens);
    if (variant >= p.nvariants)
        return set_error(TRK_ERR_INVALID, "trk_plan_describe: no variant %d", variant);
    const Variant &v = p.variants[variant];
    const Chain &c = p.chains[v.chain];
    std::memset(info, 0, sizeof(*info));
    std::snprintf(info->name, sizeof(info->name), "%s", v.name);
    info->kind = v.kind;
    std::copy(c.order, c.order + 3, info->order);
    std::copy(v.tile, v.tile + 5, info->tile);
    grid_of(p, v, tokens, info->grid);
    info->block = v.block;
    info->lds_bytes = v.lds_bytes;
    info->t_min = v.t_min;
    info->t_max = v.t_max;
    // algorithmic work of the cores' rank (a padded plan's kernels do more, on zeros)
    info->flops = chain_flops_per_token(p, c, p.core_rank) * tokens;
    double params = 0.0;
    for (int m = 0; m < 3; ++m)
        params += double(p.core_rank) * p.core_rank * p.in_modes[m] * p.out_modes[m];
    info->bytes = double(p.elem) * (params + double(tokens) * (p.in_features + p.out_features));
    info->packed_offset[0] = c.offF;
    info->packed_offset[1] = c.offS;
    info->packed_offset[2] = c.offL;
    return TRK_OK;
}

int trk_plan_set_variant(trk_plan *plan, int t_min, int t_max, int variant) {
    if (!plan) return set_error(TRK_ERR_INVALID, "trk_plan_set_variant: null plan");
    Plan &p = *as_plan(plan);
    if (variant < 0 || variant >= p.nvariants || t_min < 1 || t_max < t_min)
        return set_error(TRK_ERR_INVALID, "trk_plan_set_variant: bad variant or token range");
    // Take [t_min, t_max] out of every other variant's range (a range that would split in
    // two keeps its lower part), then give it to `variant`, whose old range it replaces.
    // Variant 0 (generic) serves every count no other range covers.
    for (int i = 1; i < p.nvariants; ++i) {
        Variant &v = p.variants[i];
        if (i == variant || v.t_min <= 0) continue;
        if (v.t_max < t_min || v.t_min > t_max) continue;
        if (v.t_min >= t_min && v.t_max <= t_max) {
            v.t_min = v.t_max = 0;
        } else if (v.t_min < t_min) {
            v.t_max = t_min - 1;
        } else {
            v.t_min = t_max + 1;
        }
    }
    if (variant > 0) {
        p.variants[variant].t_min = t_min;
        p.variants[variant].t_max = t_max;
    }
    return TRK_OK;
}

int trk_pack(const trk_plan *plan, const void *g1, const void *g2, const void *g3, void *packed,
             void *stream) {
    if (!plan || !g1 || !g2 || !g3 || !packed)
        return set_error(TRK_ERR_INVALID, "trk_pack: null argument");
    return launch_pack(*as_plan(plan), g1, g2, g3, packed, static_cast<hipStream_t>(stream));
}

int trk_forward_epilogue(const trk_plan *plan, int variant, const void *packed, const void *x,
                         void *y, int tokens, int epilogue, const void *aux, int aux_dtype,
                         void *stream) {
    if (!plan) return set_error(TRK_ERR_INVALID, "trk_forward: null plan");
    const Plan &p = *as_plan(plan);
    if (tokens < 0) return set_error(TRK_ERR_INVALID, "trk_forward: tokens < 0");
    if (epilogue < TRK_EPI_STORE || epilogue > TRK_EPI_SILU_MUL)
        return set_error(TRK_ERR_INVALID, "trk_forward: unknown epilogue %d", epilogue);
    const bool reads_aux = epilogue == TRK_EPI_ADD || epilogue == TRK_EPI_SILU_MUL;
    if (reads_aux && aux_dtype != p.dtype && aux_dtype != TRK_DTYPE_F32)
        return set_error(TRK_ERR_INVALID,
                         "trk_forward: aux dtype %d is neither the plan's (%d) nor fp32",
                         aux_dtype, p.dtype);
    if (variant < 0) variant = trk_plan_select(plan, tokens);
    if (variant >= p.nvariants)
        return set_error(TRK_ERR_INVALID, "trk_forward: no variant %d", variant);
    if (tokens == 0) return TRK_OK;
    if (!packed || !x || !y || (reads_aux && !aux))
        return set_error(TRK_ERR_INVALID, "trk_forward: null buffer");
    const int aux_align = reads_aux ? (aux_dtype == TRK_DTYPE_F32 ? 4 : p.elem) : 1;
    const int y_align = epilogue == TRK_EPI_F32 ? 4 : p.elem;
    if ((reinterpret_cast<uintptr_t>(aux) & (aux_align - 1)) ||
        (reinterpret_cast<uintptr_t>(y) & (y_align - 1)))
        return set_error(TRK_ERR_INVALID, "trk_forward: y or aux not aligned to its element");
    const Variant &v = p.variants[variant];
    if (v.kind == TRK_KERNEL_MFMA &&
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(packed)) & 15))
        return set_error(TRK_ERR_INVALID, "trk_forward: x and packed must be 16-byte aligned");
    Epi epi{reads_aux ? aux : nullptr,
            epilogue | (reads_aux && aux_dtype == TRK_DTYPE_F32 ? kAuxF32 : 0)};
    return v.launch(p, v, packed, x, y, tokens, epi, static_cast<hipStream_t>(stream));
}

int trk_forward_variant(const trk_plan *plan, int variant, const void *packed, const void *x,
                        void *y, int tokens, void *stream) {
    if (variant < 0) return set_error(TRK_ERR_INVALID, "trk_forward: no variant %d", variant);
    return trk_forward_epilogue(plan, variant, packed, x, y, tokens, TRK_EPI_STORE, nullptr,
                                TRK_DTYPE_F16, stream);
}

int trk_forward(const trk_plan *plan, const void *packed, const void *x, void *y, int tokens,
                void *stream) {
    if (!plan) return set_error(TRK_ERR_INVALID, "trk_forward: null plan");
    return trk_forward_variant(plan, trk_plan_select(plan, tokens), packed, x, y, tokens, stream);
}

int trk_forward_swiglu(const trk_plan *gate, const void *packed_gate, const trk_plan *up,
                       const void *packed_up, const void *x, void *y, int tokens, void *stream) {
    if (!gate || !up) return set_error(TRK_ERR_INVALID, "trk_forward_swiglu: null plan");
    const Plan &g = *as_plan(gate), &u = *as_plan(up);
    if (tokens < 0) return set_error(TRK_ERR_INVALID, "trk_forward_swiglu: tokens < 0");
    if (g.dtype != u.dtype || g.rank != u.rank || g.core_rank != u.core_rank ||
        !std::equal(g.in_modes, g.in_modes + 3, u.in_modes) ||
        !std::equal(g.out_modes, g.out_modes + 3, u.out_modes) || g.nchains != u.nchains ||
        g.packed_bytes != u.packed_bytes)
        return set_error(TRK_ERR_INVALID,
                         "trk_forward_swiglu: the gate and up plans differ in shape, dtype, rank "
                         "or packed layout");
    if (tokens == 0) return TRK_OK;
    const int variant = trk_plan_select(gate, tokens);
    if (variant < 0 || variant >= g.nvariants)
        return set_error(TRK_ERR_INVALID, "trk_forward_swiglu: no variant for %d tokens", tokens);
    const Variant &v = g.variants[variant];
    const Chain &cg = g.chains[v.chain], &cu = u.chains[v.chain];
    if (cg.offF != cu.offF || cg.offS != cu.offS || cg.offL != cu.offL)
        return set_error(TRK_ERR_INVALID, "trk_forward_swiglu: the plans' packed layouts differ");
    if (!v.launch_pair)
        return set_error(TRK_ERR_UNSUPPORTED,
                         "trk_forward_swiglu: variant %s has no fused gate/up kernel", v.name);
    if (!packed_gate || !packed_up || !x || !y)
        return set_error(TRK_ERR_INVALID, "trk_forward_swiglu: null buffer");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(packed_gate) |
         reinterpret_cast<uintptr_t>(packed_up)) & 15)
        return set_error(TRK_ERR_INVALID,
                         "trk_forward_swiglu: x and the packed buffers must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(y) & (g.elem - 1))
        return set_error(TRK_ERR_INVALID, "trk_forward_swiglu: y not aligned to its element");
    return v.launch_pair(g, v, packed_gate, packed_up, x, y, tokens,
                         static_cast<hipStream_t>(stream));
}

int trk_consume_silu_mul(const float *g, const float *u, void *out, int out_dtype, size_t n,
                         void *stream) {
    if (n > 0 && (!g || !u || !out))
        return set_error(TRK_ERR_INVALID, "trk_consume_silu_mul: null buffer");
    return launch_silu_mul(g, u, out, out_dtype, n, static_cast<hipStream_t>(stream));
}

int trk_consume_add(const void *h, const float *y, void *out, int dtype, size_t n, void *stream) {
    if (n > 0 && (!h || !y || !out))
        return set_error(TRK_ERR_INVALID, "trk_consume_add: null buffer");
    return launch_add(h, y, out, dtype, n, static_cast<hipStream_t>(stream));
}

int trk_empty_launch(void *stream) { return launch_empty(static_cast<hipStream_t>(stream)); }

int trk_empty_launch_args(void *stream) {
    return launch_empty_args(static_cast<hipStream_t>(stream));
}

int trk_empty_call(void) { return TRK_OK; }

}  // extern "C"
