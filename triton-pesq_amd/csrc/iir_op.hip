// Stand-alone IIR filter (the TritonIIR operator), forward or time reversed:
// one filter in parallel form (one scan pass), or a cascade of full biquads
// (one scan pass per section, float64 rows between the passes).
#include "iir.hpp"

namespace pesq {

template <bool kRev>
struct SingleMode {
    static constexpr int kInputs = 1;
    static constexpr int kOutputs = 1;
    static constexpr bool kRamp = false;
    static constexpr bool kReverse = kRev;
    static constexpr bool kAccumulates = false;
    static constexpr bool kB2 = false;
    using In = float;
    using Out = float;

    const float *x;
    float *y;
    int64_t len;

    __device__ __forceinline__ const float *src(int row, int) const { return x + int64_t(row) * len; }
    __device__ __forceinline__ float *dst(int row, int) const { return y + int64_t(row) * len; }
    __device__ __forceinline__ void inputs(double, const float *in, double &xa, double &xb) const {
        xa = in[0];
        xb = 0.0;
    }
    __device__ __forceinline__ void setup(int, double *, int) const {}
    __device__ __forceinline__ void compute(double, double ya, double, double &, const double *,
                                            float *out) const {
        out[0] = static_cast<float>(ya);
    }
    __device__ __forceinline__ void finish(int, int, double) const {}
};

template <int NS, bool kRev>
static int launch_single(const float *x, float *y, int64_t rows, int64_t len,
                         const IirTable *table, double *aggr, hipStream_t stream) {
    SingleMode<kRev> m{x, y, len};
    return launch_scan<NS, 0>(m, table, aggr, rows, len, true, true, stream);
}

template <bool kRev>
static int dispatch(int sections, const float *x, float *y, int64_t rows, int64_t len,
                    const IirTable *table, double *aggr, hipStream_t stream) {
    switch (sections) {
        case 1: return launch_single<1, kRev>(x, y, rows, len, table, aggr, stream);
        case 2: return launch_single<2, kRev>(x, y, rows, len, table, aggr, stream);
        case 3: return launch_single<3, kRev>(x, y, rows, len, table, aggr, stream);
        case 4: return launch_single<4, kRev>(x, y, rows, len, table, aggr, stream);
        case 5: return launch_single<5, kRev>(x, y, rows, len, table, aggr, stream);
        case 6: return launch_single<6, kRev>(x, y, rows, len, table, aggr, stream);
        case 7: return launch_single<7, kRev>(x, y, rows, len, table, aggr, stream);
        case 8: return launch_single<8, kRev>(x, y, rows, len, table, aggr, stream);
        default: break;
    }
    set_error("unsupported section count %d", sections);
    return PESQ_ERR_ARGUMENT;
}

// One pass of a cascade: a full biquad (b2 kept) from In to Out.  Passes
// between the first and the last read and write float64 rows, so that the
// cascade rounds to float32 only once, at its output.
template <bool kRev, typename TIn, typename TOut>
struct CascadeMode {
    static constexpr int kInputs = 1;
    static constexpr int kOutputs = 1;
    static constexpr bool kRamp = false;
    static constexpr bool kReverse = kRev;
    static constexpr bool kAccumulates = false;
    static constexpr bool kB2 = true;
    using In = TIn;
    using Out = TOut;

    const TIn *x;
    TOut *y;
    int64_t len;

    __device__ __forceinline__ const TIn *src(int row, int) const { return x + int64_t(row) * len; }
    __device__ __forceinline__ TOut *dst(int row, int) const { return y + int64_t(row) * len; }
    __device__ __forceinline__ void inputs(double, const TIn *in, double &xa, double &xb) const {
        xa = static_cast<double>(in[0]);
        xb = 0.0;
    }
    __device__ __forceinline__ void setup(int, double *, int) const {}
    __device__ __forceinline__ void compute(double, double ya, double, double &, const double *,
                                            TOut *out) const {
        out[0] = static_cast<TOut>(ya);
    }
    __device__ __forceinline__ void finish(int, int, double) const {}
};

template <bool kRev, typename TIn, typename TOut>
static int cascade_pass(const TIn *x, TOut *y, int64_t rows, int64_t len, const IirTable *table,
                        double *aggr, hipStream_t stream) {
    CascadeMode<kRev, TIn, TOut> m{x, y, len};
    return launch_scan<1, 0>(m, table, aggr, rows, len, true, true, stream);
}

// passes k = 0 .. count - 1: float x -> double rows (alternating buffers) -> float y
template <bool kRev>
static int cascade(const float *x, float *y, int64_t rows, int64_t len, const IirTable *tables,
                   int count, double *aggr, double *mid, hipStream_t stream) {
    if (count == 1) return cascade_pass<kRev>(x, y, rows, len, tables, aggr, stream);
    double *buf[2] = {mid, mid + rows * len};
    if (int st = cascade_pass<kRev>(x, buf[0], rows, len, tables, aggr, stream)) return st;
    for (int k = 1; k < count - 1; ++k) {
        const int st = cascade_pass<kRev>(static_cast<const double *>(buf[(k - 1) & 1]),
                                          buf[k & 1], rows, len, tables + k, aggr, stream);
        if (st) return st;
    }
    return cascade_pass<kRev>(static_cast<const double *>(buf[(count - 2) & 1]), y, rows, len,
                              tables + count - 1, aggr, stream);
}

}  // namespace pesq

using namespace pesq;

extern "C" int pesq_iir_cascade_workspace(int64_t rows, int64_t len, int sections,
                                          size_t *bytes) {
    PESQ_CHECK_ARG(rows >= 0 && len >= 0 && bytes != nullptr, "invalid sizes");
    PESQ_CHECK_ARG(sections >= 1 && sections <= PESQ_IIR_MAX_CASCADE,
                   "a cascade has 1..%d sections", PESQ_IIR_MAX_CASCADE);
    const int64_t nblk = cdiv(len, kBlockSpan);
    PESQ_CHECK_ARG(rows * nblk < (int64_t(1) << 31), "too many rows x blocks for one launch");
    const int64_t mid = sections == 1 ? 0 : (sections == 2 ? 1 : 2) * rows * len;
    *bytes = size_t(scan_workspace_doubles(rows, nblk, 1) + mid) * sizeof(double);
    return PESQ_OK;
}

extern "C" int pesq_iir_cascade_apply(const float *x, float *y, int64_t rows, int64_t len,
                                      const void *cascade_tables, int sections, int reverse,
                                      void *workspace, hipStream_t stream) {
    PESQ_CHECK_ARG(x && y && cascade_tables && workspace, "null pointer argument");
    PESQ_CHECK_ARG(rows >= 0 && len >= 0, "invalid sizes");
    PESQ_CHECK_ARG(sections >= 1 && sections <= PESQ_IIR_MAX_CASCADE,
                   "a cascade has 1..%d sections", PESQ_IIR_MAX_CASCADE);
    if (rows == 0 || len == 0) return PESQ_OK;
    const int64_t nblk = cdiv(len, kBlockSpan);
    PESQ_CHECK_ARG(rows * nblk < (int64_t(1) << 31), "too many rows x blocks for one launch");
    const IirTable *tables = static_cast<const IirTable *>(cascade_tables);
    double *aggr = static_cast<double *>(workspace);
    double *mid = aggr + scan_workspace_doubles(rows, nblk, 1);
    return reverse ? cascade<true>(x, y, rows, len, tables, sections, aggr, mid, stream)
                   : cascade<false>(x, y, rows, len, tables, sections, aggr, mid, stream);
}

extern "C" int pesq_iir_workspace(int64_t rows, int64_t len, size_t *bytes) {
    PESQ_CHECK_ARG(rows >= 0 && len >= 0 && bytes != nullptr, "invalid sizes");
    const int64_t nblk = cdiv(len, kBlockSpan);
    PESQ_CHECK_ARG(rows * nblk < (int64_t(1) << 31), "too many rows x blocks for one launch");
    *bytes = size_t(scan_workspace_doubles(rows, nblk)) * sizeof(double);
    return PESQ_OK;
}

// The kernels are compiled per section count; the caller packed the table and
// passes its section count, so no device memory is read on the host.
extern "C" int pesq_iir_apply(const float *x, float *y, int64_t rows, int64_t len,
                                const void *iir_table, int sections, int reverse,
                                void *workspace, hipStream_t stream) {
    PESQ_CHECK_ARG(x && y && iir_table && workspace, "null pointer argument");
    PESQ_CHECK_ARG(rows >= 0 && len >= 0, "invalid sizes");
    if (rows == 0 || len == 0) return PESQ_OK;
    PESQ_CHECK_ARG(rows * cdiv(len, kBlockSpan) < (int64_t(1) << 31),
                   "too many rows x blocks for one launch");
    const IirTable *table = static_cast<const IirTable *>(iir_table);
    double *aggr = static_cast<double *>(workspace);
    return reverse ? dispatch<true>(sections, x, y, rows, len, table, aggr, stream)
                   : dispatch<false>(sections, x, y, rows, len, table, aggr, stream);
}
