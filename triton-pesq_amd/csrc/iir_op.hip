// Stand-alone IIR filter (the TritonIIR operator): one filter in parallel
// form, forward or time reversed, two kernels per call.
#include "iir.hpp"

namespace pesq {

template <bool kRev>
struct SingleMode {
    static constexpr int kInputs = 1;
    static constexpr int kOutputs = 1;
    static constexpr bool kRamp = false;
    static constexpr bool kReverse = kRev;
    static constexpr bool kAccumulates = false;

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

}  // namespace pesq

using namespace pesq;

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
