// The HIP device's graph breakers (csrc/backend/graph_breakers.h:12-14): MATMUL
// and SUM, the two ops the reference's CUDA device also runs outside the
// element-wise JIT (csrc/backend/cuda/kernels/blas/matmul.cu:119,
// csrc/backend/cuda/kernels/reduce/sum.cu:97). Each handler sets root->data to
// a new buffer shaped like root->view.shape, as the registry requires.
#include <memory>
#include <stdexcept>
#include <vector>

#include "backend/graph_breakers.h"
#include "backend/hip/hip_safe_call.h"
#include "core/memory.h"
#include "core/node.h"

namespace ormi::hip {
    // hip::matmul, the interface of cuda::matmul (csrc/backend/cuda/kernels/
    // blas/cuda_matmul.cuh:6-12) over ormi_hip_gemm, with cuda::matmul's
    // reading of the views (matmul.cu:29-68):
    //   M, K from A's last two dims, N from B's last dim;
    //   the batch is out_view's leading dims, row-major; an operand's offset
    //   for batch coordinate i is coord * stride of its own dim aligned to i
    //   from the right, and 0 where it lacks that dim or its extent is 1
    //   (broadcast);
    //   C is contiguous, batch b at b*M*N (matmul.cu:40,78).
    // cuda::matmul derives a trans flag and one leading dimension per operand
    // (matmul.cu:47-52), which covers views whose last or second-to-last
    // stride is 1; ormi_hip_gemm takes both strides of each operand as they
    // are, which gives the same product for those views and a correct one for
    // any other. Extent-1 batch dims are dropped and adjacent batch dims whose
    // strides nest are merged, to fit ORMI_GEMM_MAX_BATCH_DIMS.
    std::shared_ptr<Buffer> matmul(std::shared_ptr<Buffer> A, const TensorView& view_A, std::shared_ptr<Buffer> B,
                                   const TensorView& view_B, const TensorView& out_view) {
        const int na = (int)view_A.shape.size(), nb = (int)view_B.shape.size(), no = (int)out_view.shape.size();
        if (na < 2 || nb < 2 || no < 2) throw std::runtime_error("HIP MATMUL: operands need at least 2 dims.");
        auto out = empty(out_view.shape, DeviceEnum::HIP);

        ormi_gemm_desc d{};
        d.dtype = ORMI_DTYPE_F32;
        d.M = view_A.shape[na - 2];
        d.K = view_A.shape[na - 1];
        d.N = view_B.shape[nb - 1];
        d.a = A->ptr;
        d.a_stride_m = view_A.strides[na - 2];
        d.a_stride_k = view_A.strides[na - 1];
        d.b = B->ptr;
        d.b_stride_k = view_B.strides[nb - 2];
        d.b_stride_n = view_B.strides[nb - 1];
        d.c = static_cast<float*>(out->ptr);

        const int nbatch = no - 2;
        auto batch_stride = [nbatch](const TensorView& v, int i) -> int64_t {
            const int td = i - (nbatch - ((int)v.shape.size() - 2));
            return (td >= 0 && v.shape[td] > 1) ? v.strides[td] : 0;
        };
        std::vector<int> shape;
        std::vector<int64_t> sa, sb;
        for (int i = 0; i < nbatch; ++i) {
            if (out_view.shape[i] == 1) continue;
            shape.push_back(out_view.shape[i]);
            sa.push_back(batch_stride(view_A, i));
            sb.push_back(batch_stride(view_B, i));
        }
        for (size_t i = 0; i + 1 < shape.size();) {
            if (sa[i] == sa[i + 1] * shape[i + 1] && sb[i] == sb[i + 1] * shape[i + 1]) {
                shape[i] *= shape[i + 1];
                sa[i] = sa[i + 1];
                sb[i] = sb[i + 1];
                shape.erase(shape.begin() + i + 1);
                sa.erase(sa.begin() + i + 1);
                sb.erase(sb.begin() + i + 1);
            } else {
                ++i;
            }
        }
        if (shape.size() > ORMI_GEMM_MAX_BATCH_DIMS)
            throw std::runtime_error("HIP MATMUL: more than 4 batch dims that cannot be merged.");
        d.batch_ndim = (int)shape.size();
        for (size_t i = 0; i < shape.size(); ++i) {
            d.batch_shape[i] = shape[i];
            d.a_batch_stride[i] = sa[i];
            d.b_batch_stride[i] = sb[i];
        }
        HIP_SAFE_CALL(ormi_hip_gemm(&d));
        return out;
    }

    void matmul_handler(std::shared_ptr<Node> root) {
        root->data = hip::matmul(root->parents[0]->data, root->parents[0]->view, root->parents[1]->data,
                                 root->parents[1]->view, root->view);
    }

    // hip::sum, the interface of cuda::sum (csrc/backend/cuda/kernels/reduce/
    // cuda_sum.cuh:5-11) over ormi_hip_reduce. A dim is reduced when axes is
    // empty or names it (sum.cu:44-54; an entry that names no dim reduces
    // nothing); the output holds the kept dims contiguously, which keepdims
    // only reshapes. cuda::sum adds each buffer element into its output with
    // an atomic, decomposing the element's flat position by the view's
    // strides (sum.cu:20,39-65), which is the reduction of the view when the
    // view is contiguous; ormi_hip_reduce walks the view's coordinates, which
    // is that same reduction for contiguous views and the reduction of the
    // view for any other (transposed, expanded). Its order is fixed, so equal
    // inputs give equal bits, which atomics do not.
    std::shared_ptr<Buffer> sum(std::shared_ptr<Buffer> in_buf, const TensorView& in_view, const std::vector<int>& axes,
                                const TensorView& out_view, const bool keepdims) {
        (void)keepdims;
        const int nd = (int)in_view.shape.size();
        if (nd > ORMI_REDUCE_MAX_DIMS) throw std::runtime_error("HIP SUM: more than 8 dims.");
        auto out = empty(out_view.shape, DeviceEnum::HIP);

        std::vector<int> reduced;
        for (int d = 0; d < nd; ++d) {
            bool r = axes.empty();
            for (int ax : axes) r = r || ax == d;
            if (r) reduced.push_back(d);
        }
        if (reduced.empty() && nd > 0) {
            // Nothing is reduced: the output is the view, copied contiguously.
            ormi_map_leaf L{};
            L.ptr = in_buf->ptr;
            L.dtype = ORMI_DTYPE_F32;
            ormi_map_desc m{};
            m.ndim = nd;
            for (int d = 0; d < nd; ++d) {
                m.shape[d] = in_view.shape[d];
                L.strides[d] = in_view.strides[d];
            }
            m.num_leaves = 1;
            m.leaves = &L;
            int value = 0, dtype = ORMI_DTYPE_F32;
            void* dst = out->ptr;
            m.num_outputs = 1;
            m.output_values = &value;
            m.outputs = &dst;
            m.output_dtypes = &dtype;
            HIP_SAFE_CALL(ormi_hip_map(&m));
            return out;
        }

        ormi_reduce_desc r{};
        r.op = ORMI_REDUCE_SUM;
        r.in_dtype = ORMI_DTYPE_F32;
        r.in = in_buf->ptr;
        r.ndim = nd;
        for (int d = 0; d < nd; ++d) {
            r.shape[d] = in_view.shape[d];
            r.strides[d] = in_view.strides[d];
        }
        r.naxes = (int)reduced.size();
        for (int i = 0; i < r.naxes; ++i) r.axes[i] = reduced[i];
        r.out = out->ptr;
        HIP_SAFE_CALL(ormi_hip_reduce(&r));
        return out;
    }

    void sum_handler(std::shared_ptr<Node> root) {
        const auto& attrs = std::get<ReduceAttrs>(root->attrs);
        root->data = hip::sum(root->parents[0]->data, root->parents[0]->view, attrs.axes, root->view, attrs.keepdims);
    }

    static RegisterGraphBreaker reg_hip_matmul(DeviceEnum::HIP, ops::OpEnum::MATMUL, matmul_handler);
    static RegisterGraphBreaker reg_hip_sum(DeviceEnum::HIP, ops::OpEnum::SUM, sum_handler);
}
