"""Host-side support for the MI355X GSD-LQ decode engine: the A2 codebook,
the .gsd2 container, the native encoder binding, seeded synthetic models and
the ctypes binding of the HIP library."""
