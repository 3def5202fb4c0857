// KunlunK200 matmul surface, implemented for AMD Instinct MI355X (gfx950).
//
// This header keeps the declarations, argument meaning, defaults and class
// layouts of the matmul subset of the reference library's public header
// (reference include/kunlun/k200.h:10-37, 40-41, 62-107, 127-132, 185-224, 345-350)
// so a consumer of that subset rebuilds against this library unchanged.
// Declarations of the reference that are not on the matmul path (attention,
// Q6_K, the common Q4 ABI, KV caches) are not
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
// Completes every operation submitted to the selected device (reference k200.h:17).
int wait();
enum CopyKind { host_to_device, device_to_host, device_to_device };
// Submits a copy on the selected device; wait() completes it (reference k200.h:18-19).
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
// run in one fp16-MFMA GEMM with the SiLU * up epilogue; smaller batches run
// two GEMVs and the SwiGLU kernel. Submits; select + wait completes it.
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

// Same layout as the reference (reference k200.h:345-350): matmul submissions
// on devices 0 and 1, peer copy count and bytes.
struct Statistics {
    size_t matmuls[2];
    size_t peer_copies, peer_bytes;
};
Statistics statistics();
const char * version();

} // namespace kunlun
