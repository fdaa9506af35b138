// Euclidean VQ / RVQ kernels for codebooks of width K = 256.
#include "aq_euclid_kernels.hpp"

AQ_EUCLID_KS_TABLE(8)
