"""Grid constants of the LUMA log-space quantiser (src/luma_optimizer/config.py:23-25)."""

K_M: int = (1 << 15) - 1          # 32767: signed-int16 momentum magnitude
K_W: int = (1 << 16) - 1          # 65535: unsigned-int16 preconditioner range
SCALE_FLOOR_M: float = 1e-9       # minimum momentum scale S_m

# Launch geometry of the HIP kernels (the reference's get_kernel_config returns
# Triton launch parameters; these are the gfx950 equivalents).
CHUNK_ELEMS: int = 131072         # elements per chunk-table entry (one workgroup), at most
STEP_CHUNK_MIN: int = 16384       # shortest chunk the optimizer picks for a small tensor set
STEP_TARGET_CHUNKS: int = 2048    # workgroups a step aims for (8 per CU) before shortening chunks
THREADS_PER_BLOCK: int = 256      # four wave64 per workgroup
ELEMS_PER_THREAD: int = 8         # consecutive elements per thread per iteration


def get_kernel_config(device=None) -> dict:
    """Launch parameters of the HIP step (drop-in for config.py:35-73)."""
    return {"CHUNK_ELEMS": CHUNK_ELEMS, "STEP_CHUNK_MIN": STEP_CHUNK_MIN,
            "STEP_TARGET_CHUNKS": STEP_TARGET_CHUNKS, "THREADS_PER_BLOCK": THREADS_PER_BLOCK,
            "ELEMS_PER_THREAD": ELEMS_PER_THREAD}
