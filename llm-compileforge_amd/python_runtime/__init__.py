"""Runtime-side interfaces: the HAL contract and the HIP backend."""
