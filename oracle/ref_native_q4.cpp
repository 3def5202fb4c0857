// C entry points over the reference's own CPU oracle header
// (reference bench/native-q4-reference.h), compiled from where it lies under
// the reference checkout by oracle/Makefile into oracle/_ref/libkref.so.
// TEST INFRASTRUCTURE ONLY: it generates golden vectors and serves as the
// "reference" CPU baseline; the product never links it.
#include "native-q4-reference.h"

#include <cstdint>
#include <cstdlib>
#include <cstring>

using namespace native_q4_bench;

extern "C" {

// Seeded Q4_0 weights, their decoded F32 values and per-row max/127 scales
// (reference bench/native-q4-reference.h:20-56).
int kref_weights(int k, int n, unsigned char *q4, float *decoded, float *row_scales) {
    unsetenv("KUNLUN_Q4_WEIGHT_FILE");
    Weights weights(k, n);
    std::memcpy(q4, weights.q4.data(), weights.q4.size());
    std::memcpy(decoded, weights.decoded.data(), weights.decoded.size() * sizeof(float));
    std::memcpy(row_scales, weights.row_scales.data(), weights.row_scales.size() * sizeof(float));
    return 0;
}

// Seeded activation patterns 0..4 (reference bench/native-q4-reference.h:58-69).
int kref_input(int k, int batch, int pattern, float *x) {
    auto values = input(k, batch, pattern);
    std::memcpy(x, values.data(), values.size() * sizeof(float));
    return 0;
}

// FP64 reference on 6 OpenMP threads (reference bench/native-q4-reference.h:98-108).
int kref_reference(const float *w, const float *x, int k, int n, int batch, double *y) {
    std::vector<float> wv(w, w + (size_t)n * k), xv(x, x + (size_t)batch * k);
    auto result = reference(wv, xv, k, n, batch);
    std::memcpy(y, result.data(), result.size() * sizeof(double));
    return 0;
}

// The same call split as the reference's own bench times it
// (reference bench/native-q4-bench.cpp:22-25): the weight and input vectors
// are built once (kref_prepare), and kref_run times reference() alone on them.
struct Prepared {
    std::vector<float> w, x;
    int k, n, batch;
};

void *kref_prepare(const float *w, const float *x, int k, int n, int batch) {
    return new Prepared{std::vector<float>(w, w + (size_t)n * k), std::vector<float>(x, x + (size_t)batch * k), k, n,
                        batch};
}

int kref_run(void *handle, double *y) {
    const Prepared *p = static_cast<const Prepared *>(handle);
    auto result = reference(p->w, p->x, p->k, p->n, p->batch);
    if (y) std::memcpy(y, result.data(), result.size() * sizeof(double));
    return 0;
}

void kref_release(void *handle) { delete static_cast<Prepared *>(handle); }

// Multi-component per-tensor activation quantization: codes [components][batch*k]
// and component scales max/limit (reference bench/native-q4-reference.h:70-97).
int kref_activation(const float *x, int k, int batch, int bits, int components,
                    int8_t *linear, float *scales) {
    std::vector<float> xv(x, x + (size_t)batch * k);
    Activation activation(xv, k, batch, bits, components, false, false);
    std::memcpy(linear, activation.linear.data(), activation.linear.size());
    for (int part = 0; part < components; ++part) scales[part] = activation.scale[part];
    return 0;
}

}
