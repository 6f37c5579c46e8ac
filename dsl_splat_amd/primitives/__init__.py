"""Scans, radix sorting, tile ranges and SH on the HIP library."""
