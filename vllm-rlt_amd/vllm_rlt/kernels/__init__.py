"""gfx950 kernels of the paged KV path, loaded lazily from the C-ABI library."""
