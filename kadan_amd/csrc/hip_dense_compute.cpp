// Host C++ layer (placeholder until the DenseCompute mirror lands).
#include "kadan_amd.h"
