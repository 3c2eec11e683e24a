/*
 * A C host program against the C ABI of include/trk.h: what a binding in another language
 * sees. Built and run by tests/test_api_cpu.py::test_c_program_uses_the_abi (gcc, no GPU
 * needed: only the host-side entry points and argument checks are exercised).
 *
 * Prints one line per check ("ok <what>") and exits non-zero on the first failure.
 */
#include <stdio.h>
#include <string.h>

#include "trk.h"

#define CHECK(cond, what)                                                       \
    do {                                                                        \
        if (!(cond)) {                                                          \
            printf("FAIL %s (last error: %s)\n", what, trk_last_error());      \
            return 1;                                                           \
        }                                                                       \
        printf("ok %s\n", what);                                                \
    } while (0)

int main(void) {
    CHECK(trk_abi_version() == TRK_ABI_VERSION, "abi version");
    CHECK(trk_empty_call() == TRK_OK, "empty call");

    const int in_modes[3] = {8, 12, 20}, out_modes[3] = {12, 10, 24};
    trk_plan *plan = NULL;
    CHECK(trk_plan_create(in_modes, out_modes, 8, TRK_DTYPE_F16, &plan) == TRK_OK && plan,
          "plan create");
    CHECK(trk_plan_packed_bytes(plan) >= 2u * 44544u, "packed bytes cover the factors");
    CHECK(trk_plan_variant_count(plan) >= 2, "variants");

    trk_variant_info info;
    memset(&info, 0, sizeof(info));
    CHECK(trk_plan_describe(plan, -1, 1, &info) == TRK_OK, "describe T=1");
    CHECK(info.kind == TRK_KERNEL_MFMA, "MFMA kernel at T=1");
    /* 2 * (in*oF*R^2 + nS*nL*oF*oS*R^3 + nL*out*R^2) for the chain order described */
    CHECK(info.flops > 3.0e7 && info.flops < 4.1e7, "flops of one token");
    CHECK(info.bytes == 2.0 * (44544.0 + 1920.0 + 2880.0), "compulsory bytes of one token");
    CHECK(info.lds_bytes > 0 && info.lds_bytes <= 160 * 1024, "LDS within 160 KB");
    CHECK(trk_plan_select(plan, 1) >= 0 && trk_plan_select(plan, 1000) >= 0, "select");

    /* argument errors are reported, not crashed on; nothing is launched */
    CHECK(trk_forward(plan, NULL, NULL, NULL, 0, NULL) == TRK_OK, "tokens == 0 launches nothing");
    CHECK(trk_forward(plan, NULL, NULL, NULL, -1, NULL) == TRK_ERR_INVALID, "negative tokens");
    CHECK(trk_forward(plan, NULL, NULL, NULL, 1, NULL) == TRK_ERR_INVALID, "null buffers");
    CHECK(strstr(trk_last_error(), "null buffer") != NULL, "error message");
    CHECK(trk_forward_epilogue(plan, -1, NULL, NULL, NULL, 1, 9, NULL, TRK_DTYPE_F16, NULL) ==
              TRK_ERR_INVALID,
          "unknown epilogue");
    CHECK(trk_forward_variant(plan, 999, NULL, NULL, NULL, 1, NULL) == TRK_ERR_INVALID,
          "unknown variant");
    CHECK(trk_plan_set_variant(plan, 1, 4, 999) == TRK_ERR_INVALID, "set unknown variant");
    CHECK(trk_consume_silu_mul(NULL, NULL, NULL, TRK_DTYPE_BF16, 0, NULL) == TRK_OK,
          "empty consumer");
    CHECK(trk_consume_add(NULL, NULL, NULL, TRK_DTYPE_BF16, 4, NULL) == TRK_ERR_INVALID,
          "consumer null buffers");
    CHECK(trk_pack(plan, NULL, NULL, NULL, NULL, NULL) == TRK_ERR_INVALID, "pack null buffers");

    trk_plan *bad = NULL;
    const int zero_modes[3] = {8, 0, 20};
    CHECK(trk_plan_create(zero_modes, out_modes, 8, TRK_DTYPE_F16, &bad) == TRK_ERR_INVALID &&
              bad == NULL,
          "zero mode rejected");
    CHECK(trk_plan_create(in_modes, out_modes, 8, 7, &bad) == TRK_ERR_INVALID, "bad dtype");

    /* padded plans: rank 4 cores on the rank-8 kernels; the work reported stays rank 4's */
    trk_plan *padded = NULL, *small = NULL;
    CHECK(trk_plan_create_padded(in_modes, out_modes, 8, 4, TRK_DTYPE_F16, &bad) ==
              TRK_ERR_INVALID && bad == NULL,
          "kernel rank below the cores' rank rejected");
    CHECK(trk_plan_create_padded(in_modes, out_modes, 4, 8, TRK_DTYPE_F16, &padded) == TRK_OK,
          "padded plan");
    CHECK(trk_plan_create(in_modes, out_modes, 4, TRK_DTYPE_F16, &small) == TRK_OK, "rank-4 plan");
    trk_variant_info pinfo, sinfo;
    CHECK(trk_plan_describe(padded, -1, 1, &pinfo) == TRK_OK &&
              trk_plan_describe(small, 0, 1, &sinfo) == TRK_OK,
          "describe padded and unpadded");
    CHECK(pinfo.kind == TRK_KERNEL_MFMA, "the padded plan runs the rank-8 MFMA kernels");
    CHECK(pinfo.bytes == sinfo.bytes && pinfo.flops < info.flops, "padded plan reports rank 4's work");
    CHECK(trk_plan_packed_bytes(padded) == trk_plan_packed_bytes(plan), "sections of the kernel rank");
    int added = -1;
    CHECK(trk_plan_load_module(padded, "/nonexistent/module.so", &added) == TRK_ERR_INVALID &&
              added == 0 && strlen(trk_last_error()) > 0,
          "a missing module is an error");
    CHECK(trk_plan_load_module(padded, NULL, NULL) == TRK_ERR_INVALID, "null module path");
    trk_plan_destroy(padded);
    trk_plan_destroy(small);

    trk_plan_destroy(plan);
    trk_plan_destroy(NULL);
    printf("all checks passed\n");
    return 0;
}
