// tests/sanitize/abi_check.cpp -- drives the host side of libt81_hip's C ABI under
// AddressSanitizer + UndefinedBehaviorSanitizer (built by tests/sanitize/Makefile).
//
// Every entry point is called with arguments its checks must reject -- negative and
// extreme sizes (INT64_MIN / INT64_MAX, so that any unguarded size arithmetic overflows
// and UBSan aborts), NULL and misaligned pointers, bad dtypes, thresholds and modes --
// and the return code and error text are checked.  On a machine without a GPU, calls
// whose arguments pass every check then stop at the device check (T81_HIP_EHIP or
// T81_HIP_ENODEV); those run only when no device is present, because their pointers are
// host memory.  Exit status 0: every case returned what it should, with no sanitizer
// report (a report aborts the process).
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "t81_hip.h"

namespace {

int g_failures = 0;
int g_cases = 0;

void expect(const char *name, int rc, std::initializer_list<int> want, const char *text = nullptr) {
    ++g_cases;
    bool ok = false;
    for (int w : want) ok = ok || rc == w;
    const std::string msg = t81_hip_last_error();
    if (ok && text != nullptr && msg.find(text) == std::string::npos) ok = false;
    if (ok && rc != T81_HIP_OK && msg.empty()) ok = false;  // every failure carries text
    if (!ok) {
        ++g_failures;
        std::fprintf(stderr, "FAIL %s: rc=%d msg=\"%s\"\n", name, rc, msg.c_str());
    }
}

constexpr int64_t kMax = INT64_MAX;
constexpr int64_t kMin = INT64_MIN;

}  // namespace

int main() {
    alignas(256) static uint8_t buf[1 << 16];
    void *p = buf;                 // aligned host memory standing in for any buffer
    void *odd = buf + 1;           // misaligned for everything wider than a byte
    uint8_t *u8 = buf;
    float *f = reinterpret_cast<float *>(buf);
    const float nan = std::nanf("");
    const int no_device = t81_hip_available() == 0;
    const auto dev = {T81_HIP_EHIP, T81_HIP_ENODEV};

    // ---- K1 quantize + pack, quantize, column pack ----
    // C++ form (python/bindings.cpp:419-421): "thr <= 0 || thr > 1" rejects; NaN compares
    // false both ways and is accepted there, so it is accepted here too (below, no device)
    for (float thr : {0.0f, -0.5f, 1.5f, INFINITY})
        expect("quantize_pack thr", t81_hip_quantize_pack(p, T81_DTYPE_F32, u8, 4, 4, thr,
                                                          T81_THR_CPP, nullptr),
               {T81_HIP_EINVAL_THRESHOLD}, "threshold");
    for (float thr : {-0.1f, 1.01f, nan})
        expect("quantize_pack torch thr",
               t81_hip_quantize_pack(p, T81_DTYPE_F32, u8, 4, 4, thr, T81_THR_TORCH, nullptr),
               {T81_HIP_EINVAL_THRESHOLD});
    expect("quantize_pack mode", t81_hip_quantize_pack(p, 0, u8, 4, 4, 0.5f, 7, nullptr),
           {T81_HIP_EINVAL_THRESHOLD}, "mode");
    for (int64_t r : {int64_t{-1}, kMin})
        expect("quantize_pack rows", t81_hip_quantize_pack(p, 0, u8, r, 4, 0.5f, 0, nullptr),
               {T81_HIP_EINVAL_SHAPE});
    expect("quantize_pack cols", t81_hip_quantize_pack(p, 0, u8, 4, kMin, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("quantize_pack dtype", t81_hip_quantize_pack(p, T81_DTYPE_I8, u8, 4, 4, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_DTYPE});
    expect("quantize_pack null", t81_hip_quantize_pack(nullptr, 0, u8, 4, 4, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("quantize_pack misaligned", t81_hip_quantize_pack(odd, 0, u8, 4, 4, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("quantize count", t81_hip_quantize(p, 0, nullptr, kMin, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("quantize null", t81_hip_quantize(p, 0, nullptr, 3, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("pack_cols shape", t81_hip_pack_cols(p, 0, u8, kMin, kMax, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("pack_cols huge", t81_hip_pack_cols(p, 0, u8, kMax, kMax, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("pack_cols dtype", t81_hip_pack_cols(p, 99, u8, 2, 2, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_DTYPE});

    // ---- unpack / validate ----
    expect("unpack negative", t81_hip_unpack(u8, nullptr, -1, 1, 1, nullptr), {T81_HIP_EINVAL_SHAPE});
    expect("unpack capacity", t81_hip_unpack(u8, nullptr, 2, 1, 49, nullptr), {T81_HIP_EINVAL_SHAPE},
           "capacity");
    expect("unpack huge limbs", t81_hip_unpack(u8, nullptr, 2, kMax, 49, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("unpack huge cols", t81_hip_unpack(u8, reinterpret_cast<int8_t *>(p), 2, kMax / 47, kMax,
                                              nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("quantize_pack huge", t81_hip_quantize_pack(p, 0, u8, kMax / 2, kMax / 2, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("quantize huge", t81_hip_quantize(p, 0, reinterpret_cast<int8_t *>(p), kMax, 0.5f, 0,
                                             nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("validate huge", t81_hip_validate_packed(u8, kMax, reinterpret_cast<int32_t *>(p), nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("tq_dequantize huge", t81_hip_tq_dequantize(u8, f, kMax, kMax, T81_TQ2_0, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("validate count", t81_hip_validate_packed(u8, kMin, nullptr, nullptr), {T81_HIP_EINVAL_SHAPE});
    expect("validate null", t81_hip_validate_packed(u8, 4, nullptr, nullptr), {T81_HIP_EINVAL_POINTER});

    // ---- K2 / K3 ternary matmul ----
    auto mm = [&](int which, const void *x, int dt, const void *w, void *c, int64_t m, int64_t n,
                  int64_t k, float a, float b, const float *bias, void *ws, int64_t wsb) {
        return t81_hip_ternary_matmul_ws(which, x, dt, static_cast<const uint8_t *>(w), c, m, n, k,
                                         a, b, bias, ws, wsb, nullptr);
    };
    for (int64_t v : {int64_t{-1}, kMin})
        expect("matmul negative", mm(0, p, 1, p, p, v, 4, 4, 1, 0, nullptr, nullptr, 0),
               {T81_HIP_EINVAL_SHAPE}, "non-negative");
    for (int64_t v : {kMax, int64_t{INT_MAX}})
        expect("matmul huge m", mm(0, p, 1, p, p, v, 4, 4, 1, 0, nullptr, nullptr, 0),
               {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("matmul huge n", mm(0, p, 1, p, p, 4, kMax, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_SHAPE});
    expect("matmul huge k", mm(0, p, 1, p, p, 4, 4, kMax, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_SHAPE});
    expect("matmul dtype", mm(0, p, 7, p, p, 4, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_DTYPE});
    expect("matmul int8 alpha", mm(0, p, T81_DTYPE_I8, p, p, 4, 4, 4, 2, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_DTYPE}, "int8");
    expect("matmul int8 beta", mm(0, p, T81_DTYPE_I8, p, p, 4, 4, 4, 1, 0.5f, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_DTYPE});
    expect("matmul int8 bias", mm(0, p, T81_DTYPE_I8, p, p, 4, 4, 4, 1, 0, f, nullptr, 0),
           {T81_HIP_EINVAL_DTYPE});
    expect("matmul int8 long k", mm(0, p, T81_DTYPE_I8, p, p, 4, 4, 131072, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_SHAPE});
    expect("matmul null x", mm(0, nullptr, 1, p, p, 4, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul null w", mm(0, p, 1, nullptr, p, 4, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul null c", mm(0, p, 1, p, nullptr, 4, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul w align", mm(0, p, 1, buf + 8, p, 4, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_POINTER}, "16-byte");
    expect("matmul x align", mm(0, odd, 1, p, p, 4, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul bias align", mm(0, p, 1, p, p, 4, 4, 4, 1, 0,
                                   reinterpret_cast<const float *>(buf + 2), nullptr, 0),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul gemv m", mm(2, p, 1, p, p, 17, 4, 4, 1, 0, nullptr, nullptr, 0),
           {T81_HIP_EINVAL_SHAPE}, "M <= 16");
    expect("matmul which", mm(5, p, 1, p, p, 4, 4, 4, 1, 0, nullptr, nullptr, 0), {T81_HIP_EINVAL_SHAPE});
    expect("matmul ws size", mm(3, p, 1, p, p, 64, 4, 4, 1, 0, nullptr, nullptr, 64),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul ws negative", mm(3, p, 1, p, p, 64, 4, 4, 1, 0, nullptr, p, kMin),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul ws align", mm(3, p, 1, p, p, 64, 4, 4, 1, 0, nullptr, buf + 4, 64),
           {T81_HIP_EINVAL_POINTER});
    expect("matmul_kernel which", t81_hip_ternary_matmul_kernel(0, p, 1, u8, p, 4, 4, 4, 1, 0,
                                                                nullptr, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("noalloc negative", t81_hip_ternary_matmul_noalloc(0, p, 1, u8, p, kMin, 4, 4, 1, 0,
                                                              nullptr, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("noalloc huge", t81_hip_ternary_matmul_noalloc(3, p, 1, u8, p, 64, kMax, kMax, 1, 0,
                                                          nullptr, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    for (int64_t v : {kMin, int64_t{-1}, int64_t{0}, int64_t{16}})
        if (t81_hip_ternary_matmul_workspace_size(v, 1024, 1024, T81_DTYPE_BF16) != 0) {
            ++g_failures;
            std::fprintf(stderr, "FAIL workspace_size(%lld): expected 0\n", (long long)v);
        }
    ++g_cases;
    for (int64_t v : {kMax, kMin})
        (void)t81_hip_ternary_matmul_workspace_size(64, v, v, T81_DTYPE_BF16);  // no UB, any value
    ++g_cases;

    // ---- K4 limb GEMM and the reference activation pipeline ----
    expect("limb negative", t81_hip_gemm_ternary_limb(u8, u8, f, INT_MIN, 4, 48, 1, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "non-negative");
    expect("limb k48", t81_hip_gemm_ternary_limb(u8, u8, f, 4, 4, INT_MAX, 1, 0, nullptr),
           {T81_HIP_EINVAL_K48}, "divisible by 48");
    expect("limb empty", t81_hip_gemm_ternary_limb(nullptr, nullptr, nullptr, 0, 4, 48, 1, 0, nullptr),
           {T81_HIP_OK});
    expect("limb null", t81_hip_gemm_ternary_limb(u8, nullptr, f, 4, 4, 48, 1, 0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("limb align", t81_hip_gemm_ternary_limb(buf + 4, u8, f, 4, 4, 48, 1, 0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("mi_ref thr", t81_hip_matmul_input_reference(u8, p, 0, f, 4, 4, 48, 2.0f, 1, 0, nullptr),
           {T81_HIP_EINVAL_THRESHOLD});
    expect("mi_ref huge", t81_hip_matmul_input_reference(u8, p, 0, f, kMax, kMax, kMax, 0.5f, 1, 0,
                                                         nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("mi_ref negative", t81_hip_matmul_input_reference(u8, p, 0, f, kMin, 4, 48, 0.5f, 1, 0,
                                                             nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("mi_ref dtype", t81_hip_matmul_input_reference(u8, p, T81_DTYPE_I8, f, 4, 4, 48, 0.5f, 1,
                                                          0, nullptr),
           {T81_HIP_EINVAL_DTYPE});

    // ---- elementwise ops, transpose, GGUF ----
    expect("where n", t81_hip_where(f, f, f, f, kMin, nullptr), {T81_HIP_EINVAL_SHAPE});
    expect("where null", t81_hip_where(f, nullptr, f, f, 4, nullptr), {T81_HIP_EINVAL_POINTER});
    expect("clamp align", t81_hip_clamp(reinterpret_cast<float *>(buf + 2), f, 4, 0, 1, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("lerp n", t81_hip_lerp(f, f, f, f, -1, nullptr), {T81_HIP_EINVAL_SHAPE});
    expect("addcmul null", t81_hip_addcmul(f, f, nullptr, 1, f, 4, nullptr), {T81_HIP_EINVAL_POINTER});
    expect("transpose huge", t81_hip_transpose_packed(u8, u8, kMax, kMax, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("transpose negative", t81_hip_transpose_packed(u8, u8, kMin, 4, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("transpose align", t81_hip_transpose_packed(buf + 8, u8, 4, 4, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("tq bytes", t81_hip_tq_block_bytes(12), {T81_HIP_EINVAL_DTYPE});
    if (t81_hip_tq_block_bytes(T81_TQ1_0) != 54 || t81_hip_tq_block_bytes(T81_TQ2_0) != 66) {
        ++g_failures;
        std::fprintf(stderr, "FAIL tq_block_bytes values\n");
    }
    expect("tq_quantize quant", t81_hip_tq_quantize(f, u8, 4, 256, 0.5f, 0, nullptr),
           {T81_HIP_EINVAL_DTYPE});
    expect("tq_quantize shape", t81_hip_tq_quantize(f, u8, kMin, 256, 0.5f, T81_TQ2_0, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("tq_dequantize align", t81_hip_tq_dequantize(u8, reinterpret_cast<float *>(buf + 1), 4, 256,
                                                        T81_TQ1_0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("tq2_matmul huge", t81_hip_tq2_matmul(p, 1, u8, f, 4, kMax, kMax, 1, 0, nullptr, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("tq2_matmul n huge", t81_hip_tq2_matmul(p, 1, u8, f, 4, kMax, 256, 1, 0, nullptr, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("tq2_matmul negative", t81_hip_tq2_matmul(p, 1, u8, f, kMin, 4, 256, 1, 0, nullptr, nullptr),
           {T81_HIP_EINVAL_SHAPE});

    // ---- TQ1_0 row codec and its tensor payload ----
    auto *u16 = reinterpret_cast<uint16_t *>(buf);
    expect("tq1 rows negative", t81_hip_tq1_quantize_rows(f, kMin, 8, 0.45f, nullptr, nullptr, u16,
                                                          nullptr),
           {T81_HIP_EINVAL_SHAPE}, "non-negative");
    expect("tq1 rows huge", t81_hip_tq1_quantize_rows(f, kMax, kMax, 0.45f, nullptr, nullptr, u16,
                                                      nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("tq1 rows null", t81_hip_tq1_quantize_rows(nullptr, 2, 8, 0.45f, nullptr, nullptr, u16,
                                                      nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("tq1 rows align", t81_hip_tq1_quantize_rows(f, 2, 8, 0.45f, nullptr, nullptr,
                                                       reinterpret_cast<uint16_t *>(buf + 1),
                                                       nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("tq1 dequant negative", t81_hip_tq1_dequantize_rows(u16, 1, kMin, f, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "non-negative");
    expect("tq1 dequant null scales", t81_hip_tq1_dequantize_rows(u16, 1, 8, nullptr, f, nullptr),
           {T81_HIP_EINVAL_POINTER});
    if (t81_hip_tq1_payload_bytes(5, 13, 32, 0) != 2 + 5 * 4 ||
        t81_hip_tq1_payload_bytes(70, 100, 32, 1) != 3 * 10 + 70 * 26 ||
        t81_hip_tq1_payload_bytes(3, 8, kMin, 0) != 3 * 4 || t81_hip_tq1_payload_bytes(0, 8, 1, 1) != 0 ||
        t81_hip_tq1_payload_bytes(2, 8, kMax, 1) != 10 + 2 * 2) {
        ++g_failures;
        std::fprintf(stderr, "FAIL tq1_payload_bytes values\n");
    }
    expect("tq1 payload bytes huge",
           static_cast<int>(t81_hip_tq1_payload_bytes(kMax, kMax, kMax, 1)), {T81_HIP_EINVAL_SHAPE});
    expect("tq1 payload scale", t81_hip_tq1_dequantize_payload(u8, 1, 4, 8, 2, 0, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "buffer truncated while reading scale");
    expect("tq1 payload refinements", t81_hip_tq1_dequantize_payload(u8, 9, 4, 8, 2, 1, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "buffer truncated while skipping refinement bytes");
    expect("tq1 payload rows", t81_hip_tq1_dequantize_payload(u8, 13, 4, 8, 2, 1, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "buffer truncated while reading quantized rows");
    expect("tq1 payload second scale", t81_hip_tq1_dequantize_payload(u8, 6, 4, 8, 2, 0, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "buffer truncated while reading scale");
    expect("tq1 payload extreme group", t81_hip_tq1_dequantize_payload(u8, 3, 4, 8, kMax, 0, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "buffer truncated while reading quantized rows");
    expect("tq1 payload negative", t81_hip_tq1_dequantize_payload(u8, 64, kMin, 8, 2, 0, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "non-negative");
    expect("tq1 payload huge", t81_hip_tq1_dequantize_payload(u8, kMax, kMax, kMax, kMin, 1, f, nullptr),
           {T81_HIP_EINVAL_SHAPE}, "too large");
    expect("tq1 payload null", t81_hip_tq1_dequantize_payload(nullptr, 4, 1, 8, 2, 0, f, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("tq1 payload writer negative",
           t81_hip_tq1_quantize_payload(f, kMin, 4, 32, 0, 0.45f, u8, nullptr), {T81_HIP_EINVAL_SHAPE});
    expect("tq1 payload writer null",
           t81_hip_tq1_quantize_payload(f, 2, 4, 32, 0, 0.45f, nullptr, nullptr),
           {T81_HIP_EINVAL_POINTER});

    // ---- sparse ----
    t81_hip_spmm_plan *plan = nullptr;
    int64_t bad = 0;
    const auto *vals = reinterpret_cast<const int64_t *>(buf);
    const auto *idx = reinterpret_cast<const int32_t *>(buf);
    expect("spmm null plan", t81_hip_spmm_plan_create(vals, idx, idx, 1, 2, 2, nullptr, &bad, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("spmm dims", t81_hip_spmm_plan_create(vals, idx, idx, 1, INT_MIN, 2, &plan, &bad, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("spmm nnz", t81_hip_spmm_plan_create(vals, idx, idx, kMax, 2, 2, &plan, &bad, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    expect("spmm align", t81_hip_spmm_plan_create(reinterpret_cast<const int64_t *>(buf + 4), idx, idx,
                                                  1, 2, 2, &plan, &bad, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("spmm apply null", t81_hip_spmm_plan_apply(nullptr, f, f, 4, 1, 0, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("spmm info null", t81_hip_spmm_plan_info(nullptr, nullptr, nullptr, nullptr),
           {T81_HIP_EINVAL_POINTER});
    expect("spmm_simple N", t81_hip_spmm_simple(vals, idx, idx, 1, 2, 2, f, f, INT_MIN, 1, 0, nullptr),
           {T81_HIP_EINVAL_SHAPE});
    t81_hip_spmm_plan_destroy(nullptr);

    // ---- host-only helper ----
    double table[16 * 27];
    t81_hip_limb_tryte_table(table);
    if (table[13] != 0.0 || table[14] != 1.0 || table[12] != -1.0) {
        ++g_failures;
        std::fprintf(stderr, "FAIL limb_tryte_table values\n");
    }

    // ---- arguments that pass every check stop at the device check (no GPU only) ----
    if (no_device) {
        expect("quantize_pack device", t81_hip_quantize_pack(p, 0, u8, 4, 4, 0.5f, 0, nullptr), dev);
        expect("quantize_pack NaN thr", t81_hip_quantize_pack(p, 0, u8, 4, 4, nan, 0, nullptr), dev);
        expect("matmul device", mm(0, p, 1, p, p, 1, 64, 96, 1, 0, nullptr, nullptr, 0), dev);
        expect("matmul gemm device", mm(3, p, 1, p, p, 64, 64, 96, 1, 0.5f, f, nullptr, 0), dev);
        expect("noalloc device", t81_hip_ternary_matmul_noalloc(0, p, 1, u8, p, 64, 64, 96, 1, 0,
                                                                nullptr, nullptr),
               dev);
        expect("limb device", t81_hip_gemm_ternary_limb(u8, u8, f, 4, 4, 48, 1, 0, nullptr), dev);
        expect("unpack device", t81_hip_unpack(u8, reinterpret_cast<int8_t *>(p), 2, 1, 48, nullptr),
               dev);
        expect("transpose device", t81_hip_transpose_packed(u8, u8, 4, 4, nullptr), dev);
        expect("tq2 device", t81_hip_tq2_matmul(p, 1, u8, f, 1, 4, 256, 1, 0, nullptr, nullptr), dev);
        expect("spmm device", t81_hip_spmm_plan_create(vals, idx, idx, 1, 2, 2, &plan, &bad, nullptr),
               dev);
        expect("spmm_simple device", t81_hip_spmm_simple(vals, idx, idx, 1, 2, 2, f, f, 4, 1, 0,
                                                         nullptr),
               dev);
    }

    std::printf("abi_check: %d cases, %d failures%s\n", g_cases, g_failures,
                no_device ? " (no device: device-check cases included)" : "");
    return g_failures == 0 ? 0 : 1;
}
