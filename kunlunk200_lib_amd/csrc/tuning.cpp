// Knob table: environment read once, run-time overrides through the C ABI.
#include "tuning.h"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace kk {
namespace {

struct KnobName {
    Knob knob;
    const char *name;
};

constexpr KnobName kNames[] = {
    {kGemmMinBatch, "KUNLUN_GEMM_MIN_BATCH"},
    {kQ4MfmaMin, "KUNLUN_Q4_MFMA_MIN"},
    {kQ4MfmaMax, "KUNLUN_Q4_MFMA_MAX"},
    {kDenseMfmaMin, "KUNLUN_DENSE_MFMA_MIN"},
    {kDenseMfmaMax, "KUNLUN_DENSE_MFMA_MAX"},
    {kGemmTile, "KUNLUN_GEMM_TILE"},
    {kGemmBn, "KUNLUN_GEMM_BN"},
    {kGemvGeneral, "KUNLUN_GEMV_GENERAL"},
    {kI8FusedQuantLimit, "KUNLUN_I8_FUSED_QUANT_LIMIT"},
    {kQ4Bdiag, "KUNLUN_Q4_BDIAG"},
    {kDenseStream, "KUNLUN_DENSE_STREAM"},
    {kQ4StreamMin, "KUNLUN_Q4_STREAM_MIN"},
};
static_assert(sizeof(kNames) / sizeof(kNames[0]) == kKnobCount, "every knob has a name");

// "BMxWN" for the tile knob, a non-negative integer otherwise; -1 when the
// text is absent or malformed.
int parse(Knob knob, const char *text) {
    if (!text || !*text) return -1;
    if (knob == kGemmTile) {
        int bm = 0, wn = 0;
        if (std::sscanf(text, "%dx%d", &bm, &wn) != 2 || bm <= 0 || wn <= 0 || wn >= 1000) return -1;
        return bm * 1000 + wn;
    }
    char *end = nullptr;
    const long v = std::strtol(text, &end, 10);
    if (end == text || *end != '\0' || v < 0 || v > (1L << 30)) return -1;
    return static_cast<int>(v);
}

struct Table {
    std::atomic<int> value[kKnobCount];
    int from_env[kKnobCount];
    Table() {
        for (const KnobName &k : kNames) {
            from_env[k.knob] = parse(k.knob, std::getenv(k.name));
            value[k.knob].store(from_env[k.knob], std::memory_order_relaxed);
        }
    }
};

Table &table() {
    static Table t;   // initialised once, thread-safe
    return t;
}

} // namespace

int tuning(Knob knob) { return table().value[knob].load(std::memory_order_relaxed); }

} // namespace kk

extern "C" {

// Sets knob `name` (its environment variable name) from `value`, the same
// text the variable takes; a null value restores the value read from the
// environment at load. Returns 0, or -1 for an unknown name or a malformed value.
int kunlun_set_tuning(const char *name, const char *value) {
    if (!name) return -1;
    for (const kk::KnobName &k : kk::kNames) {
        if (std::strcmp(k.name, name) != 0) continue;
        kk::Table &t = kk::table();
        const int v = value ? kk::parse(k.knob, value) : t.from_env[k.knob];
        if (value && v < 0) return -1;
        t.value[k.knob].store(v, std::memory_order_relaxed);
        return 0;
    }
    return -1;
}

// Current value of knob `name` (-1 when unset), or -2 for an unknown name.
int kunlun_get_tuning(const char *name) {
    if (!name) return -2;
    for (const kk::KnobName &k : kk::kNames)
        if (std::strcmp(k.name, name) == 0) return kk::tuning(k.knob);
    return -2;
}

} // extern "C"
