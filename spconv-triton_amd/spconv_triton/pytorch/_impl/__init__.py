"""Host side of the gfx950 library: pair generation, gather-GEMM and pooling."""
