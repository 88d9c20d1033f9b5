"""MI355X-native paged KV-cache serving path (drop-in for the reference's
`serving` package). The append and paged attention run as HIP kernels from
libpagedkv.so; this package is their host side."""
