"""Host launchers of the gfx950 HIP kernels (mirrors the reference's
``kotflash/kernels`` package: forward, backward, strided/fused decode)."""
