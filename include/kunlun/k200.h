// KunlunK200 matmul surface, implemented for AMD Instinct MI355X (gfx950).
//
// This header keeps the declarations, argument meaning, defaults and class
// layouts of the matmul subset of the reference library's public header
// (reference include/kunlun/k200.h:10-37, 40-41, 62-107, 127-132, 185-335, 345-350)
// so a consumer of that subset rebuilds against this library unchanged.
// Declarations of the reference that are not on the matmul path (attention,
// Q6_K, KV caches, row gathers) are not
// declared here. matmul_swiglu has no reference counterpart (see below).
//
// Device numbering: the reference drives the two processing dies of one
// Kunlun card as devices 0 and 1. Here a device is one HIP device (one GPU);
// valid ids are [0, device_count()), at most kunlun::max_devices.
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>

namespace kunlun {

constexpr int max_devices = 8;

// Process-wide lock around device selection, allocation and submission
// (reference k200.h:10). Callers hold it around raw select/copy/wait runs.
std::recursive_mutex & runtime_mutex();
// Fail fast: print the diagnostic context and abort when status != 0
// (reference k200.h:11).
void check(int status);
// Optional borrowed tensor name; dimensions are copied (reference k200.h:13).
void diagnostic_tensor(const char * name, const int64_t * dimensions = nullptr);
// Fail fast when the condition is false (reference k200.h:14).
void require(bool condition);
int device_count(int * count);                       // reference k200.h:15
void select(int device);                             // reference k200.h:16
// Completes every operation on the selected device, the library's and any
// other HIP work of the process (hipDeviceSynchronize; reference k200.h:17).
int wait();
enum CopyKind { host_to_device, device_to_host, device_to_device };
// Copies on the selected device after the library's submitted work there and
// completes before returning, in every direction (reference k200.h:18-19).
int copy(void * dst, const void * src, size_t bytes, CopyKind kind);
// Device-to-device copy between GPUs; completes before returning (reference k200.h:20).
void peer(int dst_device, void * dst, int src_device, const void * src, size_t bytes);
void * allocate(int device, size_t bytes);           // reference k200.h:21, nullptr on failure
void release(int device, void * ptr, size_t bytes);  // reference k200.h:22
size_t allocated_bytes(int device);                  // reference k200.h:23

// RAII device allocation (reference k200.h:25-37).
class Buffer {
public:
    Buffer(int device, size_t bytes);
    ~Buffer();
    Buffer(const Buffer &) = delete;
    Buffer & operator=(const Buffer &) = delete;
    void * data() const { return ptr_; }
    size_t size() const { return bytes_; }
private:
    int device_;
    size_t bytes_;
    void * ptr_;
};

// Values match the reference enumeration (reference k200.h:40). q6_k is not
// accepted by matmul, as in the reference.
enum class WeightType { f32 = 0, f16 = 1, q4_0 = 2, rowwise_i8 = 3, q6_k = 4 };
// Elementwise operations (reference k200.h:41).
enum class ElementwiseOp { add = 0, multiply = 1, silu = 2, rms_norm = 3, scale = 4 };

struct SwiGLULayout;

// Per-call state owner: binds to the first device it is used on and owns
// lazily grown device workspaces (reference k200.h:62-88).
class Kernel {
public:
    Kernel();
    ~Kernel();
    Kernel(const Kernel &) = delete;
    Kernel & operator=(const Kernel &) = delete;
    struct Impl;
private:
    Impl * impl_;
    friend void matmul(Kernel &, int, void *, const void *, const void *, int, int, int,
                       WeightType, const float *, const float *, int);
    friend bool swiglu(Kernel &, int, void *, size_t, const void *, size_t, const void *, size_t,
                       const SwiGLULayout &);
    friend void matmul_swiglu(Kernel &, int, void *, const void *, const void *, const void *, int, int, int,
                              WeightType);
    friend void elementwise(Kernel &, int, void *, const void *, const void *, int, int, int, ElementwiseOp,
                            float);
};

// Packed rowwise INT8 weight layout (reference k200.h:90-96):
// [aligned(k*rows) int8 codes][aligned(4*rows) f32 row scales][256 B maxima].
size_t aligned(size_t bytes);
size_t packed_i8_size(int k, int rows);
float * packed_i8_scales(void * weights, int k, int rows);
float * packed_i8_maxima(void * weights, int k, int rows);
// Quantizes F32 host rows and uploads them to a caller-owned
// packed_i8_size(k, rows) device allocation. Completes before returning.
void upload_i8_rows(int device, void * weights, int k, int rows,
                    int first_row, int count, const float * input);

// W: [n,k], X: [batch,k], Y: [batch,n]. All pointers refer to device memory.
// Q4_0: 18-byte blocks (little-endian F16 scale + 16 paired 4-bit values).
// rowwise_i8 requires scales[n] and maxima[6], also in device memory.
// matmul submits work; select(device) + check(wait()) completes it.
// K must be divisible by 32, K <= 16384 (reference k200.h:98-105).
void matmul(Kernel &, int device, void * y, const void * w, const void * x,
            int k, int n, int batch, WeightType type,
            const float * scales = nullptr, const float * maxima = nullptr, int tile = 16);

// Element type of SwiGLU inputs and outputs (reference k200.h:132).
enum class InputType { f32, f16 };

// SiLU(gate) * up over `rows` rows of `width` contiguous values
// (reference k200.h:185-199). Strides are bytes between rows.
struct SwiGLULayout {
    int width, rows;
    int gate_stride, up_stride, output_stride;
    InputType type;
};
// Empty string: the layout is supported; otherwise "type", "shape", "stride"
// or "byte extent" names the first rule it breaks.
const char * swiglu_reason(const SwiGLULayout &);
// Computes SiLU(gate)*up with F32 intermediates and one final output
// rounding, and completes before returning. y may alias gate or up element
// for element (equal row strides), or hold rows disjoint from them; any other
// overlap, a span beyond the given byte sizes, misalignment, a bad device or
// a Kernel bound to another device returns false with no work submitted.
bool swiglu(Kernel &, int device, void * y, size_t y_bytes,
            const void * gate, size_t gate_bytes, const void * up, size_t up_bytes,
            const SwiGLULayout &);

// No counterpart in the reference, which computes this as two matmul calls
// followed by swiglu (or common_q4_matmul_pair then swiglu, reference
// src/q4-pair.inc:9-80): Y[batch,n] = SiLU(X W_gate^T) * (X W_up^T), F32 Y.
// w_gate and w_up are [n,k] weights of one type (f32, f16 or q4_0) and the
// arguments follow matmul's rules. At batch >= 64 (Q4_0, F16) both products
// run in one fp16-MFMA GEMM with the SiLU * up epilogue; Q4_0 at batch 1..2
// runs both matrices in one GEMV pass with the same epilogue; other batches
// run two GEMVs and the SwiGLU kernel. Submits; select + wait completes it.
void matmul_swiglu(Kernel &, int device, void * y, const void * w_gate, const void * w_up, const void * x,
                   int k, int n, int batch, WeightType type);

// F32 elementwise op over `count` values, completed before returning
// (reference k200.h:106-107): add and multiply take b of b_count == count
// values or of b_count == width values repeated every row; silu, scale
// (a * parameter) and rms_norm (each `width` row scaled by
// 1 / sqrt(mean(a^2) + parameter)) ignore b. count % width == 0,
// width <= 16384; y may equal a or b.
void elementwise(Kernel &, int device, void * y, const void * a, const void * b,
                 int count, int width, int b_count, ElementwiseOp op, float parameter = 0);

// Native Q4 layout (reference k200.h:127-131): the Q4_0 values and FP16
// block scales of an [n,k] matrix repacked as [N32 tile][K32 block][16 K
// pairs][32 rows] signed 4-bit values, then the scales [N32 tile][K32
// block][32 rows]; N is padded to 32 with zeros. Supported for
// 0 < k <= 16384, k % 32 == 0, 0 < n <= 90000000 / k.
bool native_q4_layout_supported(int k, int n);
// Bytes of the layout, 0 when unsupported.
size_t native_q4_size(int k, int n);
// Host repack of n rows of Q4_0 blocks into `destination` (bytes >=
// native_q4_size); false for an unsupported shape, a short or null buffer or
// overlapping ranges.
bool pack_native_q4(void * destination, size_t bytes, const void * q4, int k, int n);
// Packs on the host and copies to device memory `weights`; completes before
// returning. Invalid arguments abort.
void upload_native_q4(int device, void * weights, const void * q4, int k, int n);

// Empty string when the reference would take its accelerated route for this
// shape, otherwise the reference's reason (reference k200.h:200-203).
const char * native_q4_reason(int k, int n, int batch, InputType type);
// Reference k200.h:204-207. Here every call runs the same exact kernels, and
// no HBM or L3 workspace is held (both sizes are 0).
struct NativeQ4Statistics {
    size_t accelerated, fallback;
    size_t hbm_workspace_bytes, l3_workspace_bytes;
};
class NativeQ4Workspace {                            // reference k200.h:208-219
public:
    NativeQ4Workspace();
    ~NativeQ4Workspace();
    NativeQ4Workspace(const NativeQ4Workspace &) = delete;
    NativeQ4Workspace & operator=(const NativeQ4Workspace &) = delete;
    NativeQ4Statistics statistics() const;
    struct Impl;
private:
    Impl * impl_;
    friend bool native_q4_matmul(NativeQ4Workspace &, int, void *, const void *, const void *, int, int, int,
                                 InputType);
};
// Y[batch,n] = X[batch,k] W^T for W in the native layout (256-byte aligned),
// X F32 or F16, Y F32; completes before returning (reference k200.h:220-224).
// The result is exact up to a 23-bit fixed-point view of each 32-value
// activation block, on every route. Returns true where the reference returns
// true (native_q4_reason is empty and y and input are 64-byte aligned) and
// counts the call as accelerated, else false and counts a fallback. The
// workspace binds to the first device it is used on; invalid arguments or
// overlapping ranges abort.
bool native_q4_matmul(NativeQ4Workspace &, int device, void * y, const void * weights,
                      const void * input, int k, int n, int batch = 1, InputType type = InputType::f32);

// ---------------------------------------------------------------------------
// Common Q4 ABI v1 (reference k200.h:226-335): the persistent weight format
// K200_Q4_0_MICRO32_BANK16_KMAJOR (layout 1, scale order 1) of an [n,k] Q4_0
// matrix, padded to Kp = k rounded up to 512 (k < 512) or 256 and Np = n
// rounded up to 256. For output column c and K block b, the 16 bytes of
// signed nibble pairs (K 2p low, 2p+1 high) sit at
// ((c/32) * Kp/32 + b) * 512 + (c%16) * 32 + ((c%32)/16) * 16; the FP16 scales
// follow at scale_offset = Np*Kp/2 as [b][Np]. Payload Np*Kp*9/16 bytes.
struct CommonQ4Info {
    uint32_t abi_version, quant_type, layout, scale_order;
    int k, n, kp, np, device;
    size_t scale_offset, payload_bytes;
};
bool common_q4_supported(int k, int n);               // 0 < k <= 16384, 0 < n <= 32000
size_t common_q4_size(int k, int n);                  // payload bytes, 0 when unsupported

struct CommonQ4ActivationStatistics {
    size_t prepare_calls, quantized_chunks, quant_kernel_launches;
    size_t prepared_matmuls, prepared_chunks, invalidations, rejected_calls;
    size_t hbm_activation_bytes;
    uint64_t quantization_ns, preparation_ns;
};
struct CommonQ4ActivationChunk {
    const void * values; const void * scales;
    int first, rows, padded_rows, kp, components;
    size_t values_bytes, scales_bytes;
};
class CommonQ4ActivationLease;
class CommonQ4Workspace;

struct CommonQ4WeightStatistics { size_t uploads, upload_bytes; double pack_ms, upload_ms; };
class CommonQ4Weight {
public:
    // Borrowed storage must be 256-byte aligned, hold common_q4_size bytes and
    // outlive this handle and its calls; null storage allocates it here.
    CommonQ4Weight(int device, int k, int n, void * storage = nullptr, size_t bytes = 0);
    ~CommonQ4Weight();
    CommonQ4Weight(const CommonQ4Weight &) = delete;
    CommonQ4Weight & operator=(const CommonQ4Weight &) = delete;
    CommonQ4Info info() const;
    CommonQ4WeightStatistics statistics() const;
    void * data() const;
    // Packs n rows of ceil(k/32) Q4_0 blocks on the host and uploads them;
    // completes before returning.
    void upload(const void * q4, size_t bytes);
    struct Impl;
private:
    Impl * impl_;
    friend bool common_q4_matmul_pair(CommonQ4Workspace &, int, void *, void *, const CommonQ4Weight &,
                                      const CommonQ4Weight &, const CommonQ4ActivationLease &, uint64_t);
    friend void common_q4_matmul(CommonQ4Workspace &, int, void *, const CommonQ4Weight &, const void *, int,
                                 InputType);
    friend bool common_q4_matmul_shared(CommonQ4Workspace &, int, void *, const CommonQ4Weight &,
                                        const CommonQ4ActivationLease &, uint64_t);
};
struct CommonQ4Statistics {
    // Calls by route, as the reference counts them: GEMV (M = 1, two-component
    // A8), then M > 1 chunks by padded rows (8, 32, 64 with Kp <= 8192, 128
    // with Kp <= 4096, 64 above, 128 above), then the exact M = 1 route.
    size_t paths[8], calls, chunks;
    size_t hbm_workspace_bytes, l3_workspace_bytes, slice_bytes;
};
// Counters of the reference's SD engine schedules; always zero here.
struct CommonQ4MacStatistics {
    size_t baseline_sd_calls, stream_sd_calls, shape_fallbacks, resident_l1d_bytes;
};
// Device view of the last call's quantized activations (components 0: none).
// components 2 (M = 1): code of K index j at values[(j/32)*64 + j%32], the
// residual code at values[2*kp + (j/32)*64 + j%32], F32 scales[0] and [1].
// components 1 (M > 1): row r's codes at values[r*kp + j], scale scales[r*16].
struct CommonQ4Quantization { const void * values; const void * scales; int rows, kp, components; };
struct CommonQ4PairStatistics { size_t calls, declined, l3_partial_bytes; };
enum class CommonQ4PairStatus { NotAttempted, Success, Disabled, InvalidInput, Configuration, WeightAbi, Lease, Alias,
                                Workspace };
class CommonQ4Workspace {
public:
    CommonQ4Workspace();
    ~CommonQ4Workspace();
    CommonQ4Workspace(const CommonQ4Workspace &) = delete;
    CommonQ4Workspace & operator=(const CommonQ4Workspace &) = delete;
    CommonQ4Statistics statistics() const;
    CommonQ4ActivationStatistics activation_statistics() const;
    CommonQ4MacStatistics mac_statistics() const;
    // Borrowed device buffers, valid until the next call or workspace destruction.
    CommonQ4Quantization quantization() const;
    struct Impl;
private:
    Impl * impl_;
    friend CommonQ4PairStatistics common_q4_pair_statistics(const CommonQ4Workspace &);
    friend CommonQ4PairStatus common_q4_pair_last_status(const CommonQ4Workspace &);
    friend bool common_q4_matmul_pair(CommonQ4Workspace &, int, void *, void *, const CommonQ4Weight &,
                                      const CommonQ4Weight &, const CommonQ4ActivationLease &, uint64_t);
    friend void common_q4_matmul(CommonQ4Workspace &, int, void *, const CommonQ4Weight &, const void *, int,
                                 InputType);
    friend bool common_q4_prepare(CommonQ4Workspace &, int, const void *, int, int, InputType, uint64_t,
                                  CommonQ4ActivationLease &);
    friend bool common_q4_matmul_shared(CommonQ4Workspace &, int, void *, const CommonQ4Weight &,
                                        const CommonQ4ActivationLease &, uint64_t);
};
// Y[m,n] = X[m,k] W^T, X F32 or F16 contiguous, Y F32; completes before
// returning (reference k200.h:300-302). M = 1 quantizes X per tensor into two
// int8 components (the exact F32 product when Np * Kp > 2^27, as the
// reference's exact route); M > 1 quantizes each row to int8 (Row A8). The
// original weight scales are exact. Invalid arguments, another device's
// weight, overlap or misalignment abort before any launch.
void common_q4_matmul(CommonQ4Workspace &, int device, void * y, const CommonQ4Weight &,
                      const void * input, int m, InputType type = InputType::f32);

// A quantized snapshot of X for later common_q4_matmul_shared and
// common_q4_matmul_pair calls (reference k200.h:306-322). The owner passes a
// new nonzero generation after writing X; any other workspace call retires it.
class CommonQ4ActivationLease {
public:
    CommonQ4ActivationLease();
    ~CommonQ4ActivationLease();
    CommonQ4ActivationLease(const CommonQ4ActivationLease &) = delete;
    CommonQ4ActivationLease & operator=(const CommonQ4ActivationLease &) = delete;
    void reset();
    bool matches(int device, int k, int rows, InputType, uint64_t generation) const;
    size_t chunks() const;
    CommonQ4ActivationChunk chunk(size_t index) const;
    struct Impl;
private:
    Impl * impl_;
    friend bool common_q4_matmul_pair(CommonQ4Workspace &, int, void *, void *, const CommonQ4Weight &,
                                      const CommonQ4Weight &, const CommonQ4ActivationLease &, uint64_t);
    friend bool common_q4_prepare(CommonQ4Workspace &, int, const void *, int, int, InputType, uint64_t,
                                  CommonQ4ActivationLease &);
    friend bool common_q4_matmul_shared(CommonQ4Workspace &, int, void *, const CommonQ4Weight &,
                                        const CommonQ4ActivationLease &, uint64_t);
};
// False (and a rejected call counted) for an unsupported descriptor; no launch.
bool common_q4_prepare(CommonQ4Workspace &, int device, const void * input, int k, int rows,
                       InputType, uint64_t generation, CommonQ4ActivationLease &);
// False means no output was written (stale lease, wrong weight or overlap).
bool common_q4_matmul_shared(CommonQ4Workspace &, int device, void * y, const CommonQ4Weight &,
                             const CommonQ4ActivationLease &, uint64_t generation);
// Gate/up pair over one prepared M = 1 F32 lease (reference k200.h:381-383,
// src/q4-pair.inc:9-80):
// y0 = X W0^T, y1 = X W1^T for the shapes the reference accepts (K4096 x
// N11008, K2048 x N5632, unpadded); false with a status otherwise.
bool common_q4_matmul_pair(CommonQ4Workspace &, int device, void * y0, void * y1, const CommonQ4Weight & w0,
                           const CommonQ4Weight & w1, const CommonQ4ActivationLease &, uint64_t generation);
CommonQ4PairStatistics common_q4_pair_statistics(const CommonQ4Workspace &);
CommonQ4PairStatus common_q4_pair_last_status(const CommonQ4Workspace &);

// Same layout as the reference (reference k200.h:345-350): matmul submissions
// on devices 0 and 1, peer copy count and bytes.
struct Statistics {
    size_t matmuls[2];
    size_t peer_copies, peer_bytes;
};
Statistics statistics();
const char * version();

} // namespace kunlun
