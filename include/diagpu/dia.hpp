// Umbrella header of the C++ drop-in API (compile with hipcc, link -ldiagpu).
#pragma once

#include "chain.hpp"
#include "common.hpp"
#include "dia_reconstruct.hpp"
#include "gemm_diag.hpp"
#include "krylov.hpp"
#include "spgemm.hpp"
