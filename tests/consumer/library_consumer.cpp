// A C++ consumer of the public interface, built with only <kunlun/k200.h>
// and the KunlunK200::kunlunk200 CMake target. It runs the reference
// library-bench call sequence (reference bench/library-bench.cpp:102-129:
// Buffer, Kernel, upload, matmul, select + check(wait()), copy back) for
// F32, F16, Q4_0 and rowwise INT8 weights and checks Y against an FP64 dot
// product of the exactly known weights:
//   * the reference's own bound |y - gold| <= tol * (1 + |gold|), tol = 1e-3
//     (2e-2 for rowwise INT8) (reference bench/library-bench.cpp:125), for
//     every case below the fp16-MFMA GEMM (batch < 64);
//   * for F32, F16 and Q4_0 also |y - gold| <= 1e-4 * ||x|| * ||w_row||, and
//     at batch >= 64 the fp16-MFMA GEMM's 2e-3 * ||x|| * ||w_row|| alone.
// The data are this program's own: weights are exact F16 values (m / 1024,
// |m| < 64) or Q4_0 blocks with power-of-two scales, so the FP64 gold needs
// no F16 decoder. One line per case, "PASS" or "FAIL"; exit 0 when all pass.
#include <kunlun/k200.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace {

struct Lcg {   // Numerical Recipes' 32-bit LCG, top bits
    uint32_t s;
    explicit Lcg(uint32_t seed) : s(seed * 2654435761u + 1u) {}
    uint32_t next() { return (s = s * 1664525u + 1013904223u) >> 8; }
    int range(int lo, int hi) { return lo + static_cast<int>(next() % static_cast<uint32_t>(hi - lo + 1)); }
};

// F16 bits of v = m / 1024 with |m| < 2048 (exact: normal or zero).
uint16_t f16_bits(int m) {
    if (m == 0) return 0;
    const uint16_t sign = m < 0 ? 0x8000 : 0;
    unsigned a = static_cast<unsigned>(m < 0 ? -m : m);
    int e = 0;
    while ((a >> e) > 1) ++e;                                   // a = 1.f * 2^e
    const unsigned mant = (a << (10 - e)) & 0x3ffu;             // exact for e <= 10
    const unsigned exp = static_cast<unsigned>(e - 10 + 15);    // value a * 2^-10
    return static_cast<uint16_t>(sign | (exp << 10) | mant);
}

const char *type_name(kunlun::WeightType t) {
    switch (t) {
    case kunlun::WeightType::f32: return "f32";
    case kunlun::WeightType::f16: return "f16";
    case kunlun::WeightType::q4_0: return "q4_0";
    default: return "rowwise_i8";
    }
}

void put(int device, void *dst, const void *src, size_t bytes) {
    kunlun::select(device);
    kunlun::check(kunlun::copy(dst, src, bytes, kunlun::host_to_device));
    kunlun::check(kunlun::wait());
}

void get(int device, void *dst, const void *src, size_t bytes) {
    kunlun::select(device);
    kunlun::check(kunlun::copy(dst, src, bytes, kunlun::device_to_host));
    kunlun::check(kunlun::wait());
}

// One library-bench case; silu = run elementwise SiLU on Y in place after
// the matmul (the reference bench's pipeline mode).
bool run_case(kunlun::WeightType type, int k, int n, int batch, bool silu, uint32_t seed) {
    const int device = 0;
    Lcg rng(seed);
    std::vector<double> wd(static_cast<size_t>(n) * k);          // exact weight values
    std::vector<float> wf(wd.size());
    std::vector<uint16_t> wh(wd.size());
    std::vector<uint8_t> q4(static_cast<size_t>(n) * (k / 32) * 18);
    if (type == kunlun::WeightType::q4_0) {
        static const uint16_t scale_bits[4] = {0x2c00, 0x3000, 0xac00, 0x2800};   // 1/16, 1/8, -1/16, 1/32
        static const double scale_vals[4] = {0.0625, 0.125, -0.0625, 0.03125};
        for (int r = 0; r < n; ++r)
            for (int b = 0; b < k / 32; ++b) {
                uint8_t *blk = q4.data() + (static_cast<size_t>(r) * (k / 32) + b) * 18;
                const int s = rng.range(0, 3);
                std::memcpy(blk, &scale_bits[s], 2);
                for (int j = 0; j < 16; ++j) {
                    const int lo = rng.range(0, 15), hi = rng.range(0, 15);
                    blk[2 + j] = static_cast<uint8_t>(lo | (hi << 4));
                    wd[static_cast<size_t>(r) * k + b * 32 + j] = (lo - 8) * scale_vals[s];
                    wd[static_cast<size_t>(r) * k + b * 32 + 16 + j] = (hi - 8) * scale_vals[s];
                }
            }
    } else {
        for (size_t i = 0; i < wd.size(); ++i) {
            const int m = rng.range(-63, 63);
            wd[i] = m / 1024.0;
            wf[i] = static_cast<float>(wd[i]);
            wh[i] = f16_bits(m);
        }
    }
    std::vector<float> x(static_cast<size_t>(batch) * k), y(static_cast<size_t>(batch) * n);
    for (size_t j = 0; j < x.size(); ++j) x[j] = std::sin(0.013f * static_cast<float>(j) + 0.5f * seed);

    const size_t wbytes = type == kunlun::WeightType::f32   ? wf.size() * 4
                          : type == kunlun::WeightType::f16 ? wh.size() * 2
                          : type == kunlun::WeightType::q4_0 ? q4.size()
                                                             : kunlun::packed_i8_size(k, n);
    kunlun::Buffer dw(device, wbytes), dx(device, x.size() * 4), dy(device, y.size() * 4);
    kunlun::Kernel kernel;
    if (type == kunlun::WeightType::rowwise_i8)
        kunlun::upload_i8_rows(device, dw.data(), k, n, 0, n, wf.data());
    else
        put(device, dw.data(),
            type == kunlun::WeightType::f32   ? static_cast<const void *>(wf.data())
            : type == kunlun::WeightType::f16 ? static_cast<const void *>(wh.data())
                                              : static_cast<const void *>(q4.data()),
            wbytes);
    put(device, dx.data(), x.data(), x.size() * 4);
    const bool i8 = type == kunlun::WeightType::rowwise_i8;
    for (int rep = 0; rep < 3; ++rep) {   // the same Kernel reused, as the reference bench does
        kunlun::matmul(kernel, device, dy.data(), dw.data(), dx.data(), k, n, batch, type,
                       i8 ? kunlun::packed_i8_scales(dw.data(), k, n) : nullptr,
                       i8 ? kunlun::packed_i8_maxima(dw.data(), k, n) : nullptr);
        kunlun::select(device);
        kunlun::check(kunlun::wait());
        if (silu)
            kunlun::elementwise(kernel, device, dy.data(), dy.data(), dy.data(), n * batch, n, n * batch,
                                kunlun::ElementwiseOp::silu);
    }
    kunlun::select(device);
    kunlun::check(kunlun::wait());
    get(device, y.data(), dy.data(), y.size() * 4);

    // each rep recomputes Y = X W^T before the in-place SiLU: Y = SiLU(X W^T)
    bool ok = true;
    double max_abs = 0, err2 = 0, energy = 0, worst_ratio = 0;
    for (int b = 0; b < batch; ++b) {
        double xn = 0;
        for (int j = 0; j < k; ++j) xn += double(x[static_cast<size_t>(b) * k + j]) * x[static_cast<size_t>(b) * k + j];
        for (int r = 0; r < n; ++r) {
            double gold = 0, wn = 0;
            for (int j = 0; j < k; ++j) {
                const double w = wd[static_cast<size_t>(r) * k + j];
                gold += w * x[static_cast<size_t>(b) * k + j];
                wn += w * w;
            }
            if (silu) gold = gold / (1.0 + std::exp(-gold));
            const double v = y[static_cast<size_t>(b) * n + r], diff = std::fabs(v - gold);
            const double tol = i8 ? 0.02 : 0.001;
            const bool gemm = !i8 && batch >= 64;   // its contract is the relative bound below
            ok = ok && std::isfinite(v) && (gemm || diff <= tol * (1.0 + std::fabs(gold)));
            if (!i8 && !silu) {   // fp16-MFMA GEMM from batch 64: its 2e-3 relative bound
                const double bound = (batch >= 64 ? 2e-3 : 1e-4) * std::sqrt(xn) * std::sqrt(wn);
                ok = ok && diff <= bound;
                if (bound > 0) worst_ratio = std::max(worst_ratio, diff / bound);
            }
            max_abs = std::max(max_abs, diff);
            err2 += (v - gold) * (v - gold);
            energy += gold * gold;
        }
    }
    std::printf("matmul%s format=%s k=%d n=%d batch=%d max_abs=%g nmse=%g err/bound=%g %s\n", silu ? "+silu" : "",
                type_name(type), k, n, batch, max_abs, err2 / std::max(energy, 1e-30), worst_ratio,
                ok ? "PASS" : "FAIL");
    std::fflush(stdout);
    return ok;
}

} // namespace

int main() {
    std::lock_guard<std::recursive_mutex> lock(kunlun::runtime_mutex());
    int devices = 0;
    kunlun::check(kunlun::device_count(&devices));
    std::printf("KunlunK200 %s, %d device(s)\n", kunlun::version(), devices);
    if (devices < 1) return 1;
    struct Case { kunlun::WeightType type; int k, n, batch; bool silu; };
    const Case cases[] = {
        {kunlun::WeightType::f32, 256, 65, 4, false},    {kunlun::WeightType::f16, 256, 65, 4, false},
        {kunlun::WeightType::q4_0, 256, 65, 4, false},   {kunlun::WeightType::rowwise_i8, 256, 65, 4, false},
        {kunlun::WeightType::f32, 4096, 4096, 1, false}, {kunlun::WeightType::f16, 4096, 4096, 1, false},
        {kunlun::WeightType::q4_0, 4096, 4096, 1, false}, {kunlun::WeightType::rowwise_i8, 1024, 512, 4, false},
        {kunlun::WeightType::q4_0, 1024, 512, 64, false}, {kunlun::WeightType::f32, 256, 65, 4, true},
    };
    const size_t before = kunlun::allocated_bytes(0);
    bool all = true;
    uint32_t seed = 1;
    for (const Case &c : cases) all = run_case(c.type, c.k, c.n, c.batch, c.silu, seed++) && all;
    const size_t after = kunlun::allocated_bytes(0);
    std::printf("buffers released: %s\n", after == before ? "yes" : "no");
    all = all && after == before;
    std::printf("%s\n", all ? "ALL PASS" : "SOME FAILED");
    return all ? 0 : 1;
}
