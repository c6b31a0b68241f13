// Hand-written MFMA contraction template for gfx950 (filled in by the GEMM work).
#pragma once
