"""Outlined group names and the entry points that run them (no imports: the
decision pipeline reads this table without loading any library)."""

# Outlined-function name (without the _<idx> suffix) -> entry point.  The
# names are the outliner's (OutlineFusedGroupsPass.cpp:69-82): short names for
# matmul, conv2d (NCHW), fill and generic, the op name with dots replaced for
# every other op.  A tensor.pad that feeds a group's convolution is not in the
# group (the outliner unites linalg producers only, :140-144); the entry point
# folds it.  The inverted residual block outlines as two groups -- expand,
# then depthwise + project + residual after the pad -- which one entry point
# runs together (npu_amd.lower).
OUTLINED_NAMES = {
    "fused_fill_matmul_generic": "fused_matmul_bias_act",
    "fused_fill_linalg_conv_2d_nhwc_fhwc_generic": "fused_conv2d_nhwc_bias_act",
    "fused_fill_linalg_depthwise_conv_2d_nhwc_hwc_generic_fill_linalg_conv_2d_nhwc_fhwc_generic":
        "fused_irb_f32",
}
