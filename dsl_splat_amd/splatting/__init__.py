"""Projected-splat geometry, camera preparation and tile binning."""
