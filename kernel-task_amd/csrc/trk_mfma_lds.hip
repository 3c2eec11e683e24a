// Variant table of the ring3_mfma kernels that keep the first- and second-core slices in LDS
// (small token counts).
#include "trk_mfma_kernel.h"

namespace trk {
namespace {

// tile(shape, TT, FC, SC, LC, IC, stage-3 KS3, NACC[, WIDE (the waves splitting the stage-2
// rows), stage-2 MFMA edge]), default token range (0 0: reachable by index only)
const Entry kEntries[] = {
    // 1920 -> 2880, (8,12,20) -> (12,10,24), rank 8, fp16, chain (G3, G2, G1)
    TRK_ENTRY(tile(kR8, 1, 1, 2, 12, 8, 1, 4), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 2, 12, 8, 4, 1), 1, 1)
    TRK_ENTRY(tile(kR8, 1, 1, 2, 12, 8, 8, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 2, 12, 8, 4, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 1, 12, 8, 8, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 4, 12, 8, 8, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 2, 12, 8, 2, 2), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 1, 12, 8, 1, 4), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 5, 12, 8, 1, 4), 0, 0)
    TRK_ENTRY(tile(kR8, 1, 1, 10, 12, 8, 1, 4), 2, 1 << 30)
    TRK_ENTRY(tile(kR8, 1, 2, 5, 12, 8, 1, 4), 0, 0)
    TRK_ENTRY(tile(kR8, 4, 1, 10, 12, 4, 2, 1), 0, 0)
    // same modes, rank 16, fp16
    TRK_ENTRY(tile(kR16, 1, 1, 1, 12, 4, 2, 2), 0, 0)
    TRK_ENTRY(tile(kR16, 1, 1, 1, 12, 4, 4, 1), 0, 0)
    TRK_ENTRY(tile(kR16, 1, 1, 1, 12, 4, 8, 1, 0, 16, 8), 1, 1)
    TRK_ENTRY(tile(kR16, 1, 1, 2, 12, 4, 4, 1), 0, 0)
    TRK_ENTRY(tile(kR16, 1, 1, 5, 12, 4, 1, 4), 0, 0)
    TRK_ENTRY(tile(kR16, 1, 1, 10, 12, 2, 1, 4), 0, 0)
    // 4096 -> 14336, (16,16,16) -> (16,28,32), rank 8, bf16, chain (G1, G2, G3)
    TRK_ENTRY(tile(kUp, 1, 1, 2, 32, 8, 2, 2), 1, 1)
    TRK_ENTRY(tile(kUp, 1, 1, 2, 32, 8, 4, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kUp, 1, 1, 2, 32, 8, 8, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kUp, 1, 1, 2, 32, 8, 4, 1), 0, 0)
    TRK_ENTRY(tile(kUp, 1, 1, 4, 32, 8, 2, 2), 0, 0)
    TRK_ENTRY(tile(kUp, 1, 1, 7, 32, 8, 1, 2), 0, 0)
    TRK_ENTRY(tile(kUp, 1, 1, 14, 32, 8, 1, 2), 2, 8)
    TRK_ENTRY(tile(kUp, 1, 1, 28, 32, 8, 1, 2), 9, 64)
    // 14336 -> 4096, (16,28,32) -> (16,16,16), rank 16, bf16, chain (G3, G2, G1)
    TRK_ENTRY(tile(kDown, 1, 1, 1, 16, 2, 4, 1), 1, 1)
    TRK_ENTRY(tile(kDown, 1, 1, 1, 16, 2, 8, 1, 0, 16, 8), 0, 0)
    TRK_ENTRY(tile(kDown, 1, 1, 2, 16, 2, 4, 1), 0, 0)
};

}  // namespace

int mfma_register_lds(Plan *plan) {
    return register_entries(plan, kEntries, int(sizeof(kEntries) / sizeof(kEntries[0])));
}

}  // namespace trk
