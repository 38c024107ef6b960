"""MI355X-native drop-in for the hot path of alexkato29/high-dimensional-splatting.

`gaussian_splatting.rasterizer` (rasterize, project_gaussians, FEATURE_SLICE_WIDTH, _get_rasterizer),
`gaussian_splatting.utils.sh` (eval_sh, rgb_to_sh) and `gaussian_splatting.utils.loss` (ssim, l1_loss,
psnr) keep the reference's module paths, names and signatures; underneath, every stage runs in the
hand-written HIP library libhds_rasterizer.so through its C ABI (include/hds_rasterizer.h).
"""
