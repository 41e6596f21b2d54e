// Process-wide engine options: which implementation runs where two exist.
#pragma once

namespace mg {

enum Option : int {
    OPT_GEMM_KERNEL = 0,       // 0 automatic, 1 streaming, 2 weight-stationary
    OPT_ATTENTION_KERNEL = 1,  // 0 automatic, 1 reference order (VALU), 2 matrix cores, 3 projection fused in
    OPT_SCAN_KERNEL = 2,       // 0 automatic, 1 latch scan then rule-input packing, 2 fused
    OPT_STEP_GRAPH = 3,        // decode steps: 0 automatic (replayed from a captured HIP graph), 1 launched
                               // one kernel at a time, 2 graph
    OPT_STEP_KERNEL = 4,       // decode steps: 0 automatic, 1 layer by layer, 2 one workgroup per session
                               // (step1_kernel), 3 one workgroup per 16 sessions (tile_step_kernel),
                               // wherever the model fits them
    OPT_OPERANDS = 5,          // batched forward: 0 automatic, 1 limb planes written by a row pass before every
                               // GEMM, 2 the GLU output and the attention output read as fp32 by the GEMMs
                               // that take them (expanded to digits as they are loaded), where they fit
    OPT_KV_RINGS = 6,          // session K/V rings, chosen when a set is created: 0 automatic (packed where
                               // the decode attention kernels built on rk_head take the model), 1 fp32,
                               // 2 packed (24-bit mantissas with a power-of-two scale per row), where they fit
    OPT_COUNT
};

// Current value of an option.
int option(int opt);
// All options packed into one value (changes whenever any option does).
int options_key();
// Sets an option (value < 0 only reads it); returns the previous value, or -1 for an unknown option or
// value.
int set_option(int opt, int value);

}  // namespace mg
