// int8 instantiations of the weight-streaming matvec (one translation unit per weight type so the
// 56 kernel variants per type compile in parallel).
#include "matvec_impl.h"

namespace cllm {

template <>
void launch_matvec_wt<WType::INT8>(Epilogue ep, const MatvecArgs& a, int rpb, hipStream_t s) {
    mv::launch_wt<WType::INT8>(ep, a, rpb, s);
}

}  // namespace cllm
