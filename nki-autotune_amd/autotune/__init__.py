"""Autotune: sweep tile configs of the MI355X kernels, profile, select the fastest."""
