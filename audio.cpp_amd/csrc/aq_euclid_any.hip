// Euclidean VQ / RVQ at any codebook width and size: the exact scan with a
// run-time width, every frame of a stage scanned in the recipe's arithmetic.
#include "aq_euclid_kernels.hpp"

namespace aq_euclid {
const AnyKernels *kernels_any() {
    static const AnyKernels t = {{euclid_exact_scan_kernel<OMNI, false, 0>, euclid_exact_scan_kernel<HIGGS, false, 0>,
                                  euclid_exact_scan_kernel<DIRECT, false, 0>, euclid_exact_scan_kernel<HIGGS, true, 0>}};
    return &t;
}
}  // namespace aq_euclid
