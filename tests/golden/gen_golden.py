"""Writes the golden vectors of tests/golden/*.npz from the reference's own CPU implementation
(quantize, dequantize, MUL_MAT, R32 pack, MUL_MAT_ID, GET_ROWS).

The reference (src/core/ref/{quant,ops,f16}.cpp, src/core/{op,tensor,status}.cpp,
src/tensor/tensor.cpp and the inline R32 pack of src/backends/opencl11/r32.h) is compiled from its
sources by `make -C oracle ref` into oracle/_ref/libscrapgpu_ref.so; this script runs it on seeded
inputs and stores inputs and outputs only (no reference code travels). Run in the build container:

    make -C oracle ref && python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", ".."))
import oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def quant_inputs(dtype, rng):
    """8 blocks exercising the quantizers' branches: N(0,0.02) weights, N(0,1), a large range, an
    all-negative block (Q4_K min), an all-zero block, a constant block, tiny values, mixed signs."""
    bs = O.BLOCK[dtype]
    parts = [
        rng.standard_normal(bs) * 0.02,
        rng.standard_normal(bs),
        rng.standard_normal(bs) * 1000.0,
        -1.0 - 0.5 * np.abs(rng.standard_normal(bs)),
        np.zeros(bs),
        np.full(bs, 0.375),
        rng.standard_normal(bs) * 1e-6,
        np.where(rng.random(bs) < 0.5, -1.0, 1.0) * rng.random(bs) * 3.0,
    ]
    return np.concatenate(parts).astype(np.float32)


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libscrapgpu_ref.so is missing: run `make -C oracle ref` first")
    rng = np.random.default_rng(20261201)
    out = {}
    for dt in O.QTYPES:
        name = O.NAMES[dt]
        x = quant_inputs(dt, rng)
        q = O.ref_quantize(dt, x)
        out[f"{name}_quant_x"] = x
        out[f"{name}_quant_q"] = q
        out[f"{name}_quant_y"] = O.ref_dequantize(dt, q, x.size)
        # random block bytes: dequantization of arbitrary bit patterns (finite scales)
        nblk = 16
        raw = rng.integers(0, 256, nblk * O.TYPE_SIZE[dt], dtype=np.uint8).reshape(nblk, -1)
        scale_off = {O.Q4_0: [0], O.Q8_0: [0], O.Q4_K: [0, 2], O.Q6_K: [208]}[dt]
        for off in scale_off:
            h = (rng.integers(0x0400, 0x5000, nblk) | (rng.integers(0, 2, nblk) << 15)).astype(np.uint16)
            raw[:, off:off + 2] = h.view(np.uint8).reshape(nblk, 2)
        raw = raw.reshape(-1)
        out[f"{name}_raw_q"] = raw
        out[f"{name}_raw_y"] = O.ref_dequantize(dt, raw, nblk * O.BLOCK[dt])
        # MUL_MAT through scrapgpu_ref_execute: the GPU test shapes of tests/ops/ops_tests.cpp:702-727
        # plus ragged M and the column counts of the panel paths
        K = 256 if O.BLOCK[dt] == 256 else 96
        for M, N in ((24, 1), (24, 4), (37, 7), (37, 17)):
            w = O.ref_quantize(dt, (rng.standard_normal(K * M) * 0.02).astype(np.float32))
            xx = rng.standard_normal((N, K)).astype(np.float32)
            out[f"{name}_mm_K{K}_M{M}_N{N}_w"] = w
            out[f"{name}_mm_K{K}_M{M}_N{N}_x"] = xx
            out[f"{name}_mm_K{K}_M{M}_N{N}_y"] = O.ref_mul_mat(dt, w, K, M, xx)
        # R32 pack of the reference: 2 slices of 40 rows (one full group + a group of 8)
        Kr, Mr, S = 2 * O.BLOCK[dt], 40, 2
        nat = rng.integers(0, 256, O.row_bytes(dt, Kr) * Mr * S, dtype=np.uint8)
        out[f"{name}_r32_K{Kr}_M{Mr}_S{S}_nat"] = nat
        out[f"{name}_r32_K{Kr}_M{Mr}_S{S}_rep"] = O.ref_r32(dt, Kr, Mr, S, nat, True)
    np.savez_compressed(os.path.join(OUT, "quant_mulmat_r32.npz"), **out)
    print("wrote", len(out), "arrays")
    moe_getrows()


def moe_getrows():
    """MUL_MAT_ID (E experts, n_used slots, T tokens; x shared by the slots or one column per slot)
    and GET_ROWS (repeated, first and last rows) through scrapgpu_ref_execute."""
    rng = np.random.default_rng(20261202)
    out = {}
    for dt in O.QTYPES:
        name = O.NAMES[dt]
        K = 256 if O.BLOCK[dt] == 256 else 96
        M, E, T, nu = 40, 5, 3, 2
        w = O.ref_quantize(dt, (rng.standard_normal(K * M * E) * 0.02).astype(np.float32))
        ids = rng.integers(0, E, (T, nu)).astype(np.int32)
        ids[0, 0] = E - 1
        out[f"{name}_mid_w"] = w
        out[f"{name}_mid_ids"] = ids
        for n1 in (1, nu):
            x = rng.standard_normal((T, n1, K)).astype(np.float32)
            st, y = O.ref_mul_mat_id(dt, w, K, M, E, x, ids)
            assert st == 0, st
            out[f"{name}_mid_x{n1}"] = x
            out[f"{name}_mid_y{n1}"] = y
        R = 37
        wr = O.ref_quantize(dt, rng.standard_normal(K * R).astype(np.float32))
        rid = np.array([0, R - 1, 5, 5, 12, 30], np.int32)
        st, g = O.ref_get_rows(dt, wr, K, R, rid)
        assert st == 0, st
        out[f"{name}_gr_w"] = wr
        out[f"{name}_gr_ids"] = rid
        out[f"{name}_gr_y"] = g
    np.savez_compressed(os.path.join(OUT, "mul_mat_id_get_rows.npz"), **out)
    print("wrote", len(out), "arrays")
    float_weights()


def float_weights():
    """MUL_MAT with F32 / F16 / BF16 weights (the scalar N < 4 path, the F32 4-row panel with a
    ragged last panel, the column panels), and MUL_MAT_ID / GET_ROWS with F16 weights, through
    scrapgpu_ref_execute. Weights include values outside F16's normal range (subnormal, large)."""
    rng = np.random.default_rng(20261203)
    out = {}
    K = 72
    for dt in O.FTYPES:
        name = O.NAMES[dt]
        for M, N in ((24, 1), (23, 3), (37, 7), (37, 17)):
            wf = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
            wf[0, :4] = (3e-6, -2e-7, 900.0, -1500.0)
            w = wf if dt == O.F32 else O.float_to_half(wf) if dt == O.F16 else O.float_to_bf16(wf)
            xx = rng.standard_normal((N, K)).astype(np.float32)
            out[f"{name}_mm_K{K}_M{M}_N{N}_w"] = w
            out[f"{name}_mm_K{K}_M{M}_N{N}_x"] = xx
            out[f"{name}_mm_K{K}_M{M}_N{N}_y"] = O.ref_mul_mat(dt, w, K, M, xx)
    M, E, T, nu = 40, 5, 3, 2
    w = O.float_to_half((rng.standard_normal(K * M * E) * 0.02).astype(np.float32))
    ids = rng.integers(0, E, (T, nu)).astype(np.int32)
    out["f16_mid_w"] = w
    out["f16_mid_ids"] = ids
    x = rng.standard_normal((T, nu, K)).astype(np.float32)
    st, y = O.ref_mul_mat_id(O.F16, w, K, M, E, x, ids)
    assert st == 0, st
    out["f16_mid_x"] = x
    out["f16_mid_y"] = y
    R = 37
    wr = O.float_to_half(rng.standard_normal(K * R).astype(np.float32))
    rid = np.array([0, R - 1, 5, 5, 12, 30], np.int32)
    st, g = O.ref_get_rows(O.F16, wr, K, R, rid)
    assert st == 0, st
    out["f16_gr_w"] = wr
    out["f16_gr_ids"] = rid
    out["f16_gr_y"] = g
    np.savez_compressed(os.path.join(OUT, "float_weights.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "float":
        float_weights()
    else:
        main()
