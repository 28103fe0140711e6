// chunked prefill kernels (to come)
