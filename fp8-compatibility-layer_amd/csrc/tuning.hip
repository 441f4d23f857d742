// Tuning knobs of the kernel selection: forced tile configurations, split-K factors and routing
// thresholds, used by the sweep scripts and by the tests that force every compiled configuration.
//
// The environment is read once, when the library is loaded (a static constructor); after that a
// knob changes only through tfp8_tuning_set().  The launch path reads relaxed atomics and never
// calls getenv, so routing does not depend on environment writes made while the process runs and
// no launch pays an environment scan.
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "tfp8_common.h"

namespace tfp8 {

namespace {

struct KnobDef {
    const char* name;
    int dflt;
};

// Order matches enum Tune.  Defaults are the shipped routing (values of 0 / -1 mean "not forced").
constexpr KnobDef KNOBS[TUNE_COUNT] = {
    {"TFP8_GEMV_CFG", -1},           // streaming GEMV launch configuration id (gemv_impl.h)
    {"TFP8_GEMV_WPC", 0},            // streaming GEMV waves per CU (0: the configuration's own)
    {"TFP8_GEMV_MFMA_MIN", 4},       // smallest M for the matrix-core decode kernel
    {"TFP8_GEMV_MFMA_MAX_M", 16},    // largest M for the matrix-core decode kernel on the GEMM entry
    {"TFP8_GM_NT", 0},               // decode kernel: 16-row weight tiles per block (0: by N)
    {"TFP8_GM_W", 0},                // decode kernel: waves per block, the K split (0: by N)
    {"TFP8_GM_D", 0},                // decode kernel: chunks in flight per wave (0: by N)
    {"TFP8_GM_TL", 1},               // decode kernel: transposed (4 rows x 256 B) weight loads
    {"TFP8_GEMM_TILE", 0},           // LDS-tiled GEMM configuration index (0: by M)
    {"TFP8_GEMM_SPLITK", 0},         // split-K of the tiled and direct GEMMs (0: by shape)
    {"TFP8_GEMM_DIRECT", 1},         // direct-to-LDS GEMM enabled
    {"TFP8_GEMM_DIRECT_MIN_M", 48},  // smallest M for the direct-to-LDS GEMM
    {"TFP8_GEMM_DCFG", -1},          // direct-to-LDS GEMM configuration index (-1: by M)
    {"TFP8_GS_NW", 0},               // weight-streaming GEMM: weight tiles per wave (0: by M)
    {"TFP8_GS_KCS", 0},              // weight-streaming GEMM: 64-code chunks per step (0: by M)
    {"TFP8_GS_SPLITK", 0},           // weight-streaming GEMM split-K (0: by shape)
    {"TFP8_GS_TL", 1},               // weight-streaming GEMM: transposed weight loads
    {"TFP8_GEMM_V1", 0},             // skip the weight-streaming GEMM (LDS-tiled kernel instead)
    {"TFP8_GEMV_PAIR", 1},           // row-pair GEMV where it applies (0 off, 1 auto, 4/8 waves per block at M = 1)
    {"TFP8_GEMV_PAIR_MAX_M", 4},     // largest M (1..4) for the row-pair GEMV
    {"TFP8_GEMV_QUAD", 1},           // 4x4x4-MFMA GEMV: 0 off, 1 default (K groups up to 4 rows), 2 K groups up to 8
    {"TFP8_GEMV_QUAD_MIN_M", 3},     // smallest M for the 4x4x4-MFMA GEMV
};

std::atomic<int> g_knob[TUNE_COUNT];
int g_loaded[TUNE_COUNT];   // values in effect when the library was loaded

__attribute__((constructor)) void load_knobs() {
    for (int i = 0; i < TUNE_COUNT; ++i) {
        const char* v = getenv(KNOBS[i].name);
        g_loaded[i] = v && *v ? atoi(v) : KNOBS[i].dflt;
        g_knob[i].store(g_loaded[i], std::memory_order_relaxed);
    }
}

int find_knob(const char* name) {
    if (!name) return -1;
    for (int i = 0; i < TUNE_COUNT; ++i)
        if (!strcmp(name, KNOBS[i].name)) return i;
    return -1;
}

}  // namespace

int tune(Tune k) { return g_knob[k].load(std::memory_order_relaxed); }

}  // namespace tfp8

using namespace tfp8;

extern "C" int tfp8_tuning_set(const char* name, int value) {
    clear_error();
    const int i = find_knob(name);
    if (i < 0) return fail(TFP8_ERR_ARG, "tfp8_tuning_set: unknown knob '%s'", name ? name : "(null)");
    g_knob[i].store(value, std::memory_order_relaxed);
    return 0;
}

extern "C" int tfp8_tuning_get(const char* name, int* value) {
    clear_error();
    const int i = find_knob(name);
    if (i < 0 || !value) return fail(TFP8_ERR_ARG, "tfp8_tuning_get: unknown knob '%s'", name ? name : "(null)");
    *value = g_knob[i].load(std::memory_order_relaxed);
    return 0;
}

extern "C" void tfp8_tuning_reset(void) {
    for (int i = 0; i < TUNE_COUNT; ++i) g_knob[i].store(g_loaded[i], std::memory_order_relaxed);
}
