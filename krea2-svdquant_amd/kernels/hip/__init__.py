"""gfx950 HIP backend: ctypes binding (``lib``), torch custom ops (``ops``), backend fn (``backend``)."""
