"""Subpackage of the nnU-Net HIP inference path: resampling policy helpers."""
