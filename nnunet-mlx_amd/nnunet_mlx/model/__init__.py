"""Subpackage of the nnU-Net HIP inference path."""
