// qr_proj_api.cpp -- C ABI of the HBM-resident weight tensors and of the MLA q-absorb /
// W_UV projections (StreamingEngine.cs:517-529, :569-576).
#include <new>

#include "qr_matvec.hpp"
#include "qr_proj.hpp"
#include "qr_store.hpp"

using namespace qr;

namespace qr {

int mla_proj_prepare(MlaProjArgs& a, const void* kvb_dev, int fmt, int heads, int nope, int rope, int vdim,
                     int kv_lora) {
    QR_CHECK_ARG(kvb_dev != nullptr, "null kvb pointer");
    QR_CHECK_ARG(reinterpret_cast<uintptr_t>(kvb_dev) % 16 == 0, "kvb pointer must be 16-byte aligned");
    FormatSpec fs;
    QR_CHECK_ARG(weight_format_spec(fmt, &fs), "weight format %d is not decoded on the device", fmt);
    QR_CHECK_ARG(heads >= 1 && nope >= 1 && vdim >= 1 && rope >= 0, "bad MLA shape heads=%d nope=%d rope=%d vdim=%d",
                 heads, nope, rope, vdim);
    QR_CHECK_ARG(nope <= kMlaProjMaxNope, "nope %d above %d", nope, kMlaProjMaxNope);
    QR_CHECK_ARG(mla_proj_shape_ok(fmt, kv_lora), "kv_lora %d must be a positive multiple of 8 and of %d (format %d)",
                 kv_lora, fs.block, fmt);
    QR_CHECK_ARG(fmt != QR_FMT_Q4_K || weight_row_bytes(fmt, kv_lora) % 4 == 0, "Q4_K rows must be 4-byte multiples");
    a.w = static_cast<const uint8_t*>(kvb_dev);
    a.fmt = fmt;
    a.row_bytes = weight_row_bytes(fmt, kv_lora);
    a.heads = heads;
    a.nope = nope;
    a.rope = rope;
    a.vdim = vdim;
    a.kv_lora = kv_lora;
    return QR_OK;
}

}  // namespace qr

namespace {

bool aligned8(const void* p) { return reinterpret_cast<uintptr_t>(p) % 8 == 0; }

}  // namespace

extern "C" {

int qr_weight_row_bytes(int format, int cols, long long* out) {
    clear_error();
    QR_CHECK_ARG(out != nullptr, "null output pointer");
    const long long rb = weight_row_bytes(format, cols);
    QR_CHECK_ARG(rb >= 0, "format %d cannot hold rows of %d weights", format, cols);
    *out = rb;
    return QR_OK;
}

int qr_weight_create(qr_weight** out, int format, long long rows, int cols, const void* host_bytes) {
    clear_error();
    QR_CHECK_ARG(out != nullptr, "null output handle pointer");
    *out = nullptr;
    QR_CHECK_ARG(host_bytes != nullptr, "null weight bytes");
    QR_CHECK_ARG(rows >= 1 && cols >= 1, "bad weight shape %lld x %d", rows, cols);
    const long long rb = weight_row_bytes(format, cols);
    QR_CHECK_ARG(rb >= 0, "format %d cannot hold rows of %d weights", format, cols);
    qr_weight* w = new (std::nothrow) qr_weight();
    if (!w) {
        set_error("host allocation of the handle failed");
        return QR_ERR_OUT_OF_MEMORY;
    }
    w->format = format;
    w->rows = rows;
    w->cols = cols;
    w->row_bytes = rb;
    const size_t bytes = static_cast<size_t>(rows * rb);
    hipError_t e = hipGetDevice(&w->device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&w->dev, bytes);
    if (e == hipSuccess) e = hipMemcpy(w->dev, host_bytes, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        set_error("uploading %zu weight bytes failed: %s", bytes, hipGetErrorString(e));
        if (w->dev) (void)hipFree(w->dev);
        if (w->stream) (void)hipStreamDestroy(w->stream);
        delete w;
        return e == hipErrorOutOfMemory ? QR_ERR_OUT_OF_MEMORY : QR_ERR_HIP;
    }
    *out = w;
    return QR_OK;
}

int qr_weight_destroy(qr_weight* w) {
    clear_error();
    if (!w) return QR_OK;
    {
        DeviceGuard dg(w->device);
        if (w->dev) (void)hipFree(w->dev);
        if (w->stream) (void)hipStreamDestroy(w->stream);
        delete w;  // releases the staging buffer on the same device
    }
    return QR_OK;
}

int qr_weight_data(const qr_weight* w, const void** dev_ptr) {
    clear_error();
    QR_CHECK_ARG(w && dev_ptr, "null weight handle or output pointer");
    *dev_ptr = w->dev;
    return QR_OK;
}

int qr_mla_q_absorb_dev(const void* kvb_dev, int kvb_format, int heads, int nope, int rope, int vdim, int kv_lora,
                        int nq, const float* q_dev, float* q_tilde_dev, void* stream) {
    clear_error();
    MlaProjArgs a{};
    QR_TRY(mla_proj_prepare(a, kvb_dev, kvb_format, heads, nope, rope, vdim, kv_lora));
    QR_CHECK_ARG(nq >= 0, "negative query count");
    if (nq == 0) return QR_OK;
    QR_CHECK_ARG(q_dev && q_tilde_dev, "null q / q_tilde pointer");
    QR_CHECK_ARG(aligned8(q_tilde_dev), "q_tilde must be 8-byte aligned");
    a.nq = nq;
    a.in = q_dev;
    a.out = q_tilde_dev;
    QR_HIP(launch_mla_absorb(a, static_cast<hipStream_t>(stream)));
    return QR_OK;
}

int qr_mla_wuv_dev(const void* kvb_dev, int kvb_format, int heads, int nope, int vdim, int kv_lora, int nq,
                   const float* u_dev, float* out_dev, void* stream) {
    clear_error();
    MlaProjArgs a{};
    QR_TRY(mla_proj_prepare(a, kvb_dev, kvb_format, heads, nope, 0, vdim, kv_lora));
    QR_CHECK_ARG(nq >= 0, "negative query count");
    if (nq == 0) return QR_OK;
    QR_CHECK_ARG(u_dev && out_dev, "null u / out pointer");
    QR_CHECK_ARG(aligned8(u_dev), "u must be 8-byte aligned");
    a.nq = nq;
    a.in = u_dev;
    a.out = out_dev;
    QR_HIP(launch_mla_wuv(a, static_cast<hipStream_t>(stream)));
    return QR_OK;
}

int qr_matvec_dev(const void* w_dev, int format, long long rows, int cols, int nq, const float* x_dev,
                  float* y_dev, void* stream) {
    clear_error();
    QR_CHECK_ARG(w_dev != nullptr, "null weight pointer");
    QR_CHECK_ARG(reinterpret_cast<uintptr_t>(w_dev) % 16 == 0, "weight pointer must be 16-byte aligned");
    QR_CHECK_ARG(matvec_shape_ok(format, cols),
                 "format %d cannot take rows of %d weights (whole blocks; a multiple of 8 for F32/F16/BF16)",
                 format, cols);
    QR_CHECK_ARG(rows >= 0 && nq >= 0, "negative rows or vector count");
    QR_CHECK_ARG(nq <= 65535, "nq %d above 65535", nq);
    if (rows == 0 || nq == 0) return QR_OK;
    QR_CHECK_ARG(x_dev && y_dev, "null x / y pointer");
    QR_CHECK_ARG(reinterpret_cast<uintptr_t>(x_dev) % 16 == 0, "x must be 16-byte aligned");
    QR_CHECK_ARG(rows <= (1LL << 31) - 1, "rows %lld too large", rows);
    MatVecArgs a{};
    a.w = static_cast<const uint8_t*>(w_dev);
    a.fmt = format;
    a.rows = rows;
    a.cols = cols;
    a.row_bytes = weight_row_bytes(format, cols);
    a.nq = nq;
    a.x = x_dev;
    a.y = y_dev;
    QR_HIP(launch_matvec(a, static_cast<hipStream_t>(stream)));
    return QR_OK;
}

int qr_matvec_group_dev(int n, const void* const* w_devs, const long long* rows, int format, int cols, int nq,
                        const float* x_dev, float* const* y_devs, void* stream) {
    clear_error();
    QR_CHECK_ARG(n >= 1 && n <= kMatVecGroupMax, "group of %d matrices outside [1, %d]", n, kMatVecGroupMax);
    QR_CHECK_ARG(w_devs && rows && y_devs, "null weight / rows / y array");
    QR_CHECK_ARG(matvec_shape_ok(format, cols),
                 "format %d cannot take rows of %d weights (whole blocks; a multiple of 8 for F32/F16/BF16)",
                 format, cols);
    QR_CHECK_ARG(nq >= 0 && nq <= 65535, "nq %d outside [0, 65535]", nq);
    MatVecArgs a[kMatVecGroupMax] = {};
    int live = 0;
    for (int m = 0; m < n; ++m) {
        QR_CHECK_ARG(w_devs[m] != nullptr, "null weight pointer %d", m);
        QR_CHECK_ARG(reinterpret_cast<uintptr_t>(w_devs[m]) % 16 == 0, "weight pointer %d must be 16-byte aligned", m);
        QR_CHECK_ARG(rows[m] >= 0 && rows[m] <= (1LL << 31) - 1, "rows[%d] = %lld outside [0, 2^31)", m, rows[m]);
        if (rows[m] == 0 || nq == 0) continue;
        QR_CHECK_ARG(y_devs[m] != nullptr, "null y pointer %d", m);
        MatVecArgs& b = a[live++];
        b.w = static_cast<const uint8_t*>(w_devs[m]);
        b.fmt = format;
        b.rows = rows[m];
        b.cols = cols;
        b.row_bytes = weight_row_bytes(format, cols);
        b.nq = nq;
        b.x = x_dev;
        b.y = y_devs[m];
    }
    if (live == 0) return QR_OK;
    QR_CHECK_ARG(x_dev != nullptr, "null x pointer");
    QR_CHECK_ARG(reinterpret_cast<uintptr_t>(x_dev) % 16 == 0, "x must be 16-byte aligned");
    QR_HIP(launch_matvec_group(a, live, static_cast<hipStream_t>(stream)));
    return QR_OK;
}

int qr_matvec(const qr_weight* w, int nq, const float* x, float* y) {
    clear_error();
    QR_CHECK_ARG(w != nullptr, "null weight handle");
    QR_CHECK_ARG(nq >= 0, "negative vector count");
    if (nq == 0) return QR_OK;
    QR_CHECK_ARG(x && y, "null x / y pointer");
    QR_CHECK_ARG(matvec_shape_ok(w->format, w->cols),
                 "format %d cannot take rows of %d weights (whole blocks; a multiple of 8 for F32/F16/BF16)",
                 w->format, w->cols);
    DeviceGuard dg(w->device);
    qr_weight* mw = const_cast<qr_weight*>(w);  // staging only; the weights are not modified
    const size_t xb = static_cast<size_t>(nq) * w->cols * 4, yb = static_cast<size_t>(nq) * w->rows * 4;
    const size_t xa = (xb + 255) / 256 * 256;
    QR_TRY(mw->stage.ensure(xa + yb));
    float* dx = static_cast<float*>(mw->stage.get());
    float* dy = reinterpret_cast<float*>(static_cast<char*>(mw->stage.get()) + xa);
    QR_HIP(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, w->stream));
    QR_TRY(qr_matvec_dev(w->dev, w->format, w->rows, w->cols, nq, dx, dy, w->stream));
    QR_HIP(hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, w->stream));
    QR_HIP(hipStreamSynchronize(w->stream));
    return QR_OK;
}

}  // extern "C"
