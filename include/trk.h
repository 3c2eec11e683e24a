/*
 * trk.h - C ABI of the MI355X (gfx950) three-core tensor-ring linear operator.
 *
 *   y[t, (p,q,r)] = sum_{(i,j,k)} x[t, (i,j,k)] * sum_{a,b,c} G1[a,p,i,b] G2[b,q,j,c] G3[c,r,k,a]
 *
 * computed from the cores without ever forming the dense in x out weight.
 *
 * Conventions
 *   - Plain C types only. Device buffers are raw device pointers owned by the caller; the
 *     stream is a hipStream_t passed as void* (NULL = the null stream).
 *   - Every entry point returns an int status (TRK_OK = 0); nothing throws across the ABI.
 *     trk_last_error() returns the message of the last failure on the calling thread.
 *   - Core k is [R][o_k][i_k][R] row-major; x is [T][in] row-major; y is [T][out] row-major,
 *     with in = (i*nj + j)*nk + k and out = (p*Q + q)*Rr + r. All three share one dtype.
 *   - A plan is immutable after trk_plan_create (trk_plan_set_variant aside), so one plan
 *     may be used from several host threads and streams at once: trk_forward keeps no state
 *     between calls, allocates nothing and needs no workspace.
 *
 * The reference's native boundary is the pybind11 module of
 * src/factorized_inference/csrc/tr_ring.cu:1204-1215 plus the packing/tiling host code of
 * src/factorized_inference/tr_kernel.py; each declaration below names what it replaces.
 */
#ifndef TRK_H
#define TRK_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRK_ABI_VERSION 4

/* Element types of x, y and the cores. */
enum trk_dtype { TRK_DTYPE_F16 = 0, TRK_DTYPE_BF16 = 1, TRK_DTYPE_F32 = 2 };

/* Status codes. */
enum trk_status {
    TRK_OK = 0,
    TRK_ERR_INVALID = 1,     /* bad argument: shape, pointer, token count, variant index */
    TRK_ERR_UNSUPPORTED = 2, /* valid request that this build has no kernel for */
    TRK_ERR_HIP = 3,         /* a HIP runtime call failed (message holds hipGetErrorString) */
    TRK_ERR_NOMEM = 4        /* host allocation of the plan failed */
};

/* Kernel families. */
enum trk_kernel_kind { TRK_KERNEL_GENERIC = 0, TRK_KERNEL_MFMA = 1 };

/* What a forward call writes for each output element, with v = (TR(cores) x)[t, o] as the
 * kernel holds it (fp32 accumulator) and a = aux[t, o] (an optional [T][out] input in the
 * plan's dtype or in fp32):
 *   TRK_EPI_STORE     y[t,o] = v, in the plan's dtype (what trk_forward writes)
 *   TRK_EPI_F32       y[t,o] = v, y in fp32 (no rounding to 16 bits)
 *   TRK_EPI_ADD       y[t,o] = a + v, in the plan's dtype (residual add; aux may equal y)
 *   TRK_EPI_SILU_MUL  y[t,o] = silu(a) * v = a / (1 + exp(-a)) * v, in the plan's dtype
 *                     (the gate of a SwiGLU MLP; aux may equal y)
 * The sums are formed in fp32 and rounded once. */
enum trk_epilogue {
    TRK_EPI_STORE = 0,
    TRK_EPI_F32 = 1,
    TRK_EPI_ADD = 2,
    TRK_EPI_SILU_MUL = 3
};

typedef struct trk_plan trk_plan;

/* What one launch of a variant does (for reports, tests and roofline accounting). */
typedef struct trk_variant_info {
    char name[64];  /* kernel symbol family and tile, e.g. "ring3_mfma<CBA,1,1,2,12,8>" */
    int kind;       /* enum trk_kernel_kind */
    int order[3];   /* contraction order: first, second, last core (0 = G1, 1 = G2, 2 = G3) */
    int tile[5];    /* tokens, first-core outputs, second-core outputs, last-core outputs,
                       last-core inputs per step handled by one workgroup */
    int grid[3];    /* grid of a launch at the token count passed to trk_plan_describe */
    int block;      /* threads per workgroup */
    int lds_bytes;  /* LDS per workgroup */
    int t_min;      /* smallest token count the default selection routes here (0 = none) */
    int t_max;      /* largest token count the default selection routes here */
    double flops;   /* algorithmic flops of one launch at that token count, no padding */
    double bytes;   /* compulsory HBM bytes of one launch: cores + x + y */
    size_t packed_offset[3]; /* byte offsets in the packed buffer of the first, second and
                                last core as this variant's kernel reads them */
} trk_variant_info;

/* ABI version of the library (TRK_ABI_VERSION it was built with). No reference counterpart;
 * loaders check it before binding the other symbols. */
int trk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). Replaces the TORCH_CHECK /
 * C10_CUDA_KERNEL_LAUNCH_CHECK messages of tr_ring.cu:416-418, :1112-1115, :1160-1163. */
const char *trk_last_error(void);

/* Create a plan for one operator shape and dtype: chooses the contraction order, the kernel
 * variants per token count and the packed-core layout. Host-only (no HIP call).
 * Replaces the state set up in PreparedTRKernel.__init__ (tr_kernel.py:190-228), the tiling
 * rule choose_tiling (tr_kernel.py:118-176) and the tuned tables H100_TUNED / V3T_TILING
 * (tr_kernel.py:105-115). */
int trk_plan_create(const int in_modes[3], const int out_modes[3], int rank, int dtype,
                    trk_plan **plan);

/* trk_plan_create for cores of rank `core_rank` whose kernels run at rank `rank` >= core_rank.
 * The packed sections have the kernel rank; trk_pack fills every entry with a ring index at
 * or past core_rank with zero, so each extra term of the ring trace is zero and the result
 * is exactly that of the rank-core_rank operator. This lets ranks without compiled MFMA
 * kernels (4, 12, 24, ...) run the kernels of the next power of two. Replaces the rank
 * padding of the reference's generic WMMA kernel (tr_ring.cu:348-361, ranks padded to 16).
 * trk_variant_info.flops and .bytes stay those of the rank-core_rank operator. */
int trk_plan_create_padded(const int in_modes[3], const int out_modes[3], int core_rank,
                           int rank, int dtype, trk_plan **plan);

/* Load a variant module and add its variants to `plan`; *added (may be NULL) receives how
 * many matched the plan's shape, dtype and rank. A variant module is a shared library built
 * from a generated variant table (factorized_inference/jit.py builds one at prepare time
 * for a shape that has no compiled MFMA kernels); it is checked against this library's ABI
 * version and plan layout before it registers anything, and stays loaded for the life of
 * the process. Its variants may add packed sections, so load modules before
 * trk_plan_packed_bytes and trk_pack. Replaces the first-use build of the reference's
 * extension (tr_kernel.py:31-57, torch.utils.cpp_extension.load of tr_ring.cu). Not
 * thread-safe against other calls on the same plan. */
int trk_plan_load_module(trk_plan *plan, const char *path, int *added);

/* Free a plan (NULL is a no-op). */
void trk_plan_destroy(trk_plan *plan);

/* Bytes of the caller-owned device buffer that trk_pack fills and trk_forward reads.
 * Replaces the sizes of A1 / B2 / C3 from pack_cores (tr_kernel.py:86-99). */
size_t trk_plan_packed_bytes(const trk_plan *plan);

/* Number of kernel variants the plan holds (the default selection and every forced one). */
int trk_plan_variant_count(const trk_plan *plan);

/* Index of the variant trk_forward runs for `tokens` tokens. Replaces the per-call dispatch
 * of PreparedTRKernel.__call__ (tr_kernel.py:264-319) and v3_supported (tr_ring.cu:1099). */
int trk_plan_select(const trk_plan *plan, int tokens);

/* Describe variant `variant` (-1 = the one selected for `tokens`) at `tokens` tokens.
 * Replaces the queries smem_bytes / y_tiles / max_y_tiles (tr_ring.cu:363-372) and
 * v3t_smem (tr_ring.cu:1143-1151). */
int trk_plan_describe(const trk_plan *plan, int variant, int tokens, trk_variant_info *info);

/* Route token counts in [t_min, t_max] to `variant` from now on (tuning and tests). Replaces
 * the TR_KC / TR_TT / TR_QC / TR_V3T_TILING overrides read by tr_kernel.py:118-176,
 * :193-204. Not thread-safe against concurrent trk_forward on the same plan. */
int trk_plan_set_variant(trk_plan *plan, int t_min, int t_max, int variant);

/* Pack the three device cores into `packed` (trk_plan_packed_bytes bytes, device memory),
 * on `stream`. The cores are only read. Replaces pack_cores (tr_kernel.py:86-99). */
int trk_pack(const trk_plan *plan, const void *g1, const void *g2, const void *g3,
             void *packed, void *stream);

/* y = TR(cores) x for `tokens` rows of x, on `stream`, with the variant the plan selects.
 * x and packed are only read; y is fully written; tokens == 0 launches nothing. x and packed
 * must be 16-byte aligned (MFMA variants read them with 16-byte loads; TRK_ERR_INVALID).
 * Replaces forward / forward_v3 / forward_v3t (tr_ring.cu:448-463, :1108-1141, :1156-1192),
 * without their workspace, counters and finish pass: each output is owned by one
 * workgroup, so no cross-workgroup reduction or persistent state exists. */
int trk_forward(const trk_plan *plan, const void *packed, const void *x, void *y, int tokens,
                void *stream);

/* trk_forward with an explicit variant index (parity tests of every variant, sweeps). */
int trk_forward_variant(const trk_plan *plan, int variant, const void *packed, const void *x,
                        void *y, int tokens, void *stream);

/* trk_forward with an epilogue (enum trk_epilogue) fused into the kernel's output store, with
 * an explicit variant (-1 = the plan's selection for `tokens`). aux is [tokens][out] in
 * aux_dtype (the plan's dtype or TRK_DTYPE_F32), 16-bit aligned, read only by
 * TRK_EPI_ADD / TRK_EPI_SILU_MUL (NULL otherwise); y is fp32 for TRK_EPI_F32.
 * Replaces forward_fp32 (csrc/v3g/bind.cu:84-92, PreparedTRKernel.accumulate,
 * tr_kernel.py:230-243), which returns a view of the persistent fp32 workspace that the
 * consumer must clear; here y is an ordinary output and nothing needs clearing. TRK_EPI_ADD
 * and TRK_EPI_SILU_MUL fold consume_add / consume_silu_mul (bind.cu:96-149) into the
 * producing kernel. */
int trk_forward_epilogue(const trk_plan *plan, int variant, const void *packed, const void *x,
                         void *y, int tokens, int epilogue, const void *aux, int aux_dtype,
                         void *stream);

/* y = silu(G x) * (U x): the gate and up projections of a SwiGLU block in one launch, where
 * `gate` and `up` are plans of one shape and dtype (created alike) and packed_gate /
 * packed_up their packed cores. Each workgroup computes its tile of G x, keeps it in fp32
 * registers, computes the same tile of U x and stores silu(G x) * (U x), rounded once to the
 * dtype; nothing is allocated and no intermediate reaches memory. The variant is gate's
 * selection for `tokens`. TRK_ERR_UNSUPPORTED when that variant has no fused kernel (fused
 * kernels are compiled for the declared gate/up shapes: the Llama-3-8B up projection and the
 * Qwen3.8-27B mlp_gate_up); a caller then runs the two projections with
 * trk_forward_epilogue (TRK_EPI_F32, then TRK_EPI_SILU_MUL). Replaces the reference's
 * three-step accumulate / accumulate / consume_silu_mul chain (csrc/v3g/bind.cu:84-136),
 * which has no single-launch form. x, packed_gate and packed_up must be 16-byte aligned. */
int trk_forward_swiglu(const trk_plan *gate, const void *packed_gate, const trk_plan *up,
                       const void *packed_up, const void *x, void *y, int tokens, void *stream);

/* out[i] = silu(g[i]) * u[i] for n elements: g and u fp32, out in out_dtype (rounded once).
 * g and u are only read. Replaces consume_silu_mul (csrc/v3g/bind.cu:96-110, :126-136),
 * which also zeroes g and u because they are its persistent workspace; nothing here is
 * persistent, so nothing is cleared. */
int trk_consume_silu_mul(const float *g, const float *u, void *out, int out_dtype, size_t n,
                         void *stream);

/* out[i] = h[i] + y[i] for n elements: h and out in `dtype`, y fp32 (rounded once); out may
 * equal h. y is only read. Replaces consume_add (csrc/v3g/bind.cu:112-122, :138-149). */
int trk_consume_add(const void *h, const float *y, void *out, int dtype, size_t n, void *stream);

/* Launch floor: one empty kernel on `stream` (tr_ring.cu:1194-1200, empty_launch). */
int trk_empty_launch(void *stream);

/* Launch floor of a kernel with arguments: one empty kernel on `stream` whose argument list is
 * that of the forward kernels (56 bytes). No reference counterpart (the reference's floor
 * kernel takes no arguments): on MI355X the fetch of a launch's kernel arguments is most of
 * what a tokens=1 call costs, so this is the floor a forward call is measured against. */
int trk_empty_launch_args(void *stream);

/* Host floor: a call that does nothing (tr_ring.cu:1202, empty_call). */
int trk_empty_call(void);

#ifdef __cplusplus
}
#endif

#endif /* TRK_H */
