"""Small numeric helpers shared by the tests."""
import numpy as np


def rel_err(x, ref) -> float:
    """max |x - ref| / max |ref| (normwise max relative error)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = max(float(np.abs(ref).max()), 1e-30)
    return float(np.abs(x - ref).max()) / den


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (numpy restatement)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))
