// The repair's launches (net_ops.hip) with another piece of work's workgroups inside its first fit launch: the
// caller (api.cpp, which holds the conv plans) binds the work's arguments; gmhs_run launches round 0 through it.
#pragma once
#include "conv_kernels.h"
#include "fhc_ops.h"

namespace fhc {

struct GmCoRun {
    FitPairLaunchFn fn;   // fit round 0 with the pair's tiles (fit_pair_launcher)
    PairKArgs pk;         // the pair's arguments, pointers bound
    uint32_t tiles;       // the pair's tiles
    FitConvLaunchFn cfn;  // fit round 1 with a conv's workgroups (fit_conv_launcher), or null
    ConvKArgs ca;         // the conv's arguments, pointers bound
    dim3 cgrid;           // the conv's grid (tiles, channel tiles)
};

// fhc_gmhs with round 0 of the fit launched by co->fn beside co's pair, and round 1 by co->cfn beside co's conv
// (when given), when co is not null; fhc_gmhs_n's `pairs` pairs (co null) otherwise
int gmhs_run(const fhc_tensor* a, const fhc_tensor* b, uint32_t h, uint32_t w, const fhc_tensor* flow, uint32_t h8,
             uint32_t w8, uint32_t full_w, uint32_t level, void* ws, size_t ws_bytes, const GmCoRun* co, void* stream,
             uint32_t pairs = 1);

}  // namespace fhc
