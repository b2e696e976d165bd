/*
 * moe_gemm.hip -- prefill-path grouped expert GEMMs (MFMA).
 */
#include "dev_common.h"
#include "kernels.h"

int launch_gemm_gate_up(const ExpertSide &, const SharedSide &, const _Float16 *, int, int, int,
                        int, int, const uint32_t *, int, const uint32_t *, _Float16 *, _Float16 *,
                        hipStream_t) {
    return -2;
}
int launch_gemm_down(const ExpertSide &, const SharedSide &, const _Float16 *, const _Float16 *,
                     int, int, int, int, int, const uint32_t *, int, float *, float *, hipStream_t) {
    return -2;
}
