"""Estimator front ends (validation, allocation, launch through rl_triton._native)."""
