// Internal parameter block of the Mamba-2 SSD kernels (validated copy of
// mamba_ssd2_args, see include/mamba_hip.h).
#pragma once

#include "common.h"

namespace mamba {

struct Ssd2Params {
    int nb, L, H, P, G, N, Q, nch;
    int io_dtype;
    const void* x; int64_t x_sb, x_sl, x_sh;
    const float* dt; int64_t dt_sb, dt_sl, dt_sh;
    const float* A; const float* D;
    const void* Bm; int64_t B_sb, B_sl, B_sg;
    const void* Cm; int64_t C_sb, C_sl, C_sg;
    const float* h0; const float* init_hpr;
    void* y; int64_t y_sb, y_sl, y_sh;
    float* hT;
};

int ssd2_make_params(const mamba_ssd2_args* a, Ssd2Params* out);
size_t ssd2_generic_workspace(const Ssd2Params& p);
// ev0/ev1 (nullable hipEvent_t) are recorded around the dominant kernel.
int ssd2_generic_launch(const Ssd2Params& p, void* ws, hipStream_t stream, hipEvent_t ev0 = nullptr,
                        hipEvent_t ev1 = nullptr);

bool ssd2_mfma_supported(const Ssd2Params& p);
// heads per workgroup the MFMA scan kernel would use for p
int ssd2_mfma_hpw(const Ssd2Params& p);
size_t ssd2_mfma_workspace(const Ssd2Params& p);
int ssd2_mfma_launch(const Ssd2Params& p, void* ws, hipStream_t stream, hipEvent_t ev0 = nullptr,
                     hipEvent_t ev1 = nullptr);

}  // namespace mamba
