"""rk_matmul_t_device_noalloc (the batched products with their quantized
inputs in the library's static scratch, for callers that cannot allocate)
against rk_matmul_t_device, bit for bit, through the C-ABI: two calls in a
row, the second smaller (the array keeps the first call's contents), then
the size limit, then replays of a recorded graph."""
import ctypes

import numpy as np
import pytest

import rkhip
from oracle import oracle
from test_gpu_matvec import awkward, same_bits

pytestmark = pytest.mark.gpu

COLS = 2048
ROWS8, ROWS4 = 1000, 300


def matrices(dev, rng):
    w = awkward(rng, ROWS8 * COLS, 0.05)
    q8, s8 = oracle.quantize8(w)
    q4, s4 = oracle.quantize4(awkward(rng, ROWS4 * COLS, 0.05))
    return (q8, s8, q4, s4), [dev.upload_q8(q8, s8, ROWS8, COLS), dev.upload_q4(q4, s4, ROWS4, COLS)]


def run(dev, arena, ms, x, noalloc):
    """x [tokens][COLS] at word 0; products to the words after it; returns
    the two outputs read back."""
    tokens = x.shape[0]
    o8, o4 = tokens * COLS, tokens * COLS + tokens * ROWS8
    b = arena.begin()
    b.write(0, x.ravel())
    b.write(o8, np.full(tokens * (ROWS8 + ROWS4), np.nan, np.float32))  # stale outputs would show
    b.submit()
    call = dev.matmul_t_device_noalloc if noalloc else dev.matmul_t_device
    call(ms, [arena.device_ptr(o8), arena.device_ptr(o4)], arena.device_ptr(0), COLS, tokens)
    b = arena.begin()
    g8, g4 = b.read(o8, tokens * ROWS8), b.read(o4, tokens * ROWS4)
    b.submit()
    return np.asarray(g8).reshape(tokens, ROWS8), np.asarray(g4).reshape(tokens, ROWS4)


def test_noalloc_matches_matmul_t_device(dev):
    rng = np.random.default_rng(71)
    (q8, s8, q4, s4), ms = matrices(dev, rng)
    most = 130
    arena = dev.arena(most * (COLS + ROWS8 + ROWS4), most * (COLS + ROWS8 + ROWS4))
    try:
        for tokens in (130, 37):  # the second call smaller than the first
            x = awkward(rng, tokens * COLS, 1.0).reshape(tokens, COLS)
            want8, want4 = run(dev, arena, ms, x, noalloc=False)
            got8, got4 = run(dev, arena, ms, x, noalloc=True)
            for t in range(tokens):
                same_bits(got8[t], want8[t], f"q8 {tokens} tokens, token {t}")
                same_bits(got4[t], want4[t], f"q4 {tokens} tokens, token {t}")
            # and both are the per-token CPU products
            same_bits(got8[-1], oracle.matvec_q8(q8, s8, x[-1], ROWS8, COLS), f"q8 oracle, {tokens} tokens")
            same_bits(got4[0], oracle.matvec_q4(q4, s4, x[0], ROWS4, COLS), f"q4 oracle, {tokens} tokens")
    finally:
        arena.free()
        for m in ms:
            m.free()
    assert dev.used == 0


def test_noalloc_refuses_more_than_its_scratch(dev):
    """2^24 codes at most: 512 tokens of 32768 columns pass the check, 513
    do not, and the refusal enqueues nothing (the device stays usable)."""
    rng = np.random.default_rng(72)
    cols = 32768
    q, s = oracle.quantize8(rng.normal(0, 0.05, 16 * cols).astype(np.float32))
    m = dev.upload_q8(q, s, 16, cols)
    arena = dev.arena(64, 64)
    try:
        hs = (ctypes.c_void_p * 1)(m.h)
        outs = (ctypes.c_void_p * 1)(arena.device_ptr(0))
        rc = rkhip.lib().rk_matmul_t_device_noalloc(dev.h, 1, hs, outs, ctypes.c_void_p(arena.device_ptr(0)), cols,
                                                      513, None)
        assert rc == rkhip.RK_ERR_ARGS
        assert "static scratch" in rkhip.lib().rk_last_error(dev.h).decode()
        x = rng.normal(0, 1, cols).astype(np.float32)
        same_bits(dev.matvec(m, x), oracle.matvec_q8(q, s, x, 16, cols), "product after the refusal")
    finally:
        arena.free()
        m.free()
    assert dev.used == 0


def test_noalloc_in_a_recorded_graph(dev):
    """Recorded once into a graph and replayed: each replay gives the eager
    call's bits for the input the arena holds then (changed between
    replays by eager batches and eager products)."""
    rng = np.random.default_rng(73)
    _, ms = matrices(dev, rng)
    tokens = 70
    o8, o4 = tokens * COLS, tokens * COLS + tokens * ROWS8
    words = tokens * (COLS + ROWS8 + ROWS4)
    arena = dev.arena(2 * words, words)
    try:
        dev.graph_begin()
        dev.matmul_t_device_noalloc(ms, [arena.device_ptr(o8), arena.device_ptr(o4)], arena.device_ptr(0), COLS,
                                    tokens)
        g = dev.graph_end()
        for rep in range(3):
            x = awkward(rng, tokens * COLS, 1.0).reshape(tokens, COLS)
            want8, want4 = run(dev, arena, ms, x, noalloc=False)
            b = arena.begin()
            b.write(o8, np.full(tokens * (ROWS8 + ROWS4), np.nan, np.float32))
            b.submit()
            g.launch(1)
            b = arena.begin()
            g8, g4 = b.read(o8, tokens * ROWS8), b.read(o4, tokens * ROWS4)
            b.submit()
            g8, g4 = np.asarray(g8).reshape(tokens, ROWS8), np.asarray(g4).reshape(tokens, ROWS4)
            for t in range(tokens):
                same_bits(g8[t], want8[t], f"replay {rep} q8 token {t}")
                same_bits(g4[t], want4[t], f"replay {rep} q4 token {t}")
        g.free()
    finally:
        arena.free()
        for m in ms:
            m.free()
    assert dev.used == 0
