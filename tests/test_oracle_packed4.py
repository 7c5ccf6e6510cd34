"""Pins of the oracle's 4-bit packed backbone format (oracle.packed4_build_payload / packed4_dequant, restating
utils/pack_utils.py:126-180 and qlinear_cuda.py:2761-2786) and the host logic of the 4-bit path."""
import numpy as np
import pytest

from tris_moe_amd import ext


def _words(nibbles_per_word):
    """int32 words from lists of 8 nibbles, nibble m at bits 4m."""
    out = []
    for nib in nibbles_per_word:
        v = 0
        for m, x in enumerate(nib):
            v |= (x & 0xF) << (4 * m)
        out.append(v)
    return np.asarray(out, dtype=np.uint32).view(np.int32)


def test_known_answer_hand_derived(oracle_mod):
    """rows 8, cols 16, two groups of 8 columns: q[c][r] = c, stored zero nibble r (zero r + 1), scales 0.5 and
    2.0, so W[r][c] = (c - r - 1) * (0.5 if c < 8 else 2.0)."""
    rows, cols = 8, 16
    qweight = np.stack([np.full(rows, _words([list(range(8))])[0]),
                        np.full(rows, _words([list(range(8, 16))])[0])]).astype(np.int32)   # [2, 8]
    qzeros = np.full((2, 1), _words([list(range(8))])[0], dtype=np.int32)                  # nibble r = r
    scales = np.stack([np.full(rows, 0.5), np.full(rows, 2.0)]).astype(np.float16)
    g_idx = (np.arange(cols) // 8).astype(np.int32)
    w = oracle_mod.packed4_dequant(qweight, qzeros, scales, g_idx, rows, cols)
    assert w.shape == (8, 16) and w.dtype == np.float16
    assert w[0, 0] == -0.5 and w[3, 7] == 1.5 and w[7, 15] == 14.0 and w[7, 8] == 0.0 and w[2, 10] == 14.0
    assert w[0, 7] == 3.0 and w[7, 0] == -4.0 and w[1, 9] == 14.0 and w[6, 12] == 10.0


def test_zero_of_zero_reads_as_sixteen(oracle_mod):
    """The producer stores (round(z) - 1) & 0xF and the consumer adds one: a zero of 0 reads as 16."""
    rows, cols = 3, 8
    pl = oracle_mod.packed4_build_payload(np.zeros((rows, cols), np.float32), np.ones((1, rows), np.float32),
                                          np.zeros((1, rows), np.float32), np.zeros(cols, np.int32))
    assert (pl["qzeros"].view(np.uint32) & 0xFFF) .tolist() == [[0xFFF]]
    w = oracle_mod.packed4_dequant(pl["qweight"], pl["qzeros"], pl["scales"], pl["g_idx"], rows, cols)
    np.testing.assert_array_equal(w, np.full((rows, cols), -16.0, np.float16))


def test_exact_zero_row(oracle_mod):
    """A row of q = 1 with a stored zero nibble 0 (zero 1) dequantises to exact zeros
    (append_exact_zero_row_to_packed_4bit_payload, utils/pack_utils.py:214-250)."""
    rows, cols = 9, 12
    qweight = np.zeros((2, rows), np.int32)
    qweight[0, 8] = _words([[1] * 8])[0]
    qweight[1, 8] = _words([[1] * 4 + [0] * 4])[0]
    qzeros = np.zeros((1, 2), np.int32)
    scales = np.full((1, rows), 3.0, np.float16)
    w = oracle_mod.packed4_dequant(qweight, qzeros, scales, np.zeros(cols, np.int32), rows, cols)
    np.testing.assert_array_equal(w[8], np.zeros(cols, np.float16))
    np.testing.assert_array_equal(w[0], np.full(cols, -3.0, np.float16))   # q = 0, zero 1


@pytest.mark.parametrize("perm", [False, True], ids=["contiguous", "act_order"])
def test_quantisation_error_bound(oracle_mod, perm):
    """Round trip through the producer: |W - dequant(W)| <= s/2 (plus the fp16 rounding of the product)
    for every entry, with ragged shapes (cols % 8, rows % 8 != 0) and contiguous or permuted groups.
    A wrong nibble order, zero convention or transposition breaks the bound."""
    rng = np.random.default_rng(7)
    rows, cols, gs = 37, 90, 16
    m = rng.standard_normal((rows, cols)).astype(np.float32)
    g_idx = (np.arange(cols) // gs).astype(np.int32)
    if perm:
        g_idx = g_idx[rng.permutation(cols)]
    G = int(g_idx.max()) + 1
    lo = np.stack([m[:, g_idx == g].min(axis=1) for g in range(G)])   # [G, rows]
    hi = np.stack([m[:, g_idx == g].max(axis=1) for g in range(G)])
    scale = ((hi - lo) / 14.0).astype(np.float16).astype(np.float32)   # one step of slack for the zero's rounding
    zero = np.round(-lo / scale)
    assert zero.min() >= 1 and zero.max() <= 15   # standard normal data: min < 0 < max
    pl = oracle_mod.packed4_build_payload(m, scale, zero, g_idx)
    w = oracle_mod.packed4_dequant(pl["qweight"], pl["qzeros"], pl["scales"], pl["g_idx"], rows, cols)
    s_rc = scale[g_idx].T   # [rows, cols]
    err = np.abs(w.astype(np.float32) - m)
    bound = s_rc * 0.5 * (1 + 1e-3) + np.abs(w.astype(np.float32)) * 2.0 ** -11
    assert (err <= bound + 1e-6).all(), float((err - bound).max())


def test_uniform_group_size_detection():
    assert ext.uniform_group_size(np.arange(256) // 128) == 128
    assert ext.uniform_group_size(np.arange(260) // 32) == 32
    assert ext.uniform_group_size(np.zeros(100, np.int32)) == 104   # one group: any size >= cols
    assert ext.uniform_group_size(np.arange(96) // 12) == 0         # not a multiple of 8
    g = np.arange(256) // 128
    g[[3, 200]] = g[[200, 3]]
    assert ext.uniform_group_size(g) == 0                           # act order
    assert ext.uniform_group_size(np.arange(64) // 16 + 1) == 0     # does not start at group 0
    assert ext.uniform_group_size(np.zeros(0, np.int32)) == 0


def test_packed_matrix_module_host_state():
    """PackedQuantMatrix4bit.set_quantized keeps the reference's rows / cols defaults and the uniform group
    size (host only, no kernel calls)."""
    from tris_moe_amd.qlinear import ExpertSharedMatrix, PackedQuantMatrix4bit

    m = PackedQuantMatrix4bit()
    assert not m.is_quantized()
    rows, cols = 24, 64
    m.set_quantized(np.zeros((cols // 8, rows), np.int32), np.zeros((2, 3), np.int32),
                    np.ones((2, rows), np.float16), (np.arange(cols) // 32).astype(np.int32))
    assert m.is_quantized() and m._rows_host == rows and m._cols_host == cols and m.group_size == 32
    sm = ExpertSharedMatrix({"qweight": m.qweight, "qzeros": m.qzeros, "scales": m.scales, "g_idx": m.g_idx})
    assert sm.shared_sv_quant.is_quantized() and sm.shared_sv.numel() == 0
    sm.set_shared_sv(np.zeros((4, 8), np.float16))
    assert not sm.shared_sv_quant.is_quantized() and tuple(sm.shared_sv.shape) == (4, 8)


@pytest.mark.parametrize("rows,cols,group", [(512, 4096, 128), (37, 90, 16), (9, 8, 8)])
def test_product_packer_matches_producer(oracle_mod, rows, cols, group):
    """tris_moe_amd.packing.pack_4bit lays its payload out exactly as the oracle's restatement of the
    reference producer does for the same scales and zeros."""
    from tris_moe_amd.packing import pack_4bit

    rng = np.random.default_rng(rows + cols)
    m = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float32)
    pl = pack_4bit(m, group)
    z = (((pl["qzeros"].view(np.uint32)[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF)
         .reshape(pl["qzeros"].shape[0], -1)[:, :rows].astype(np.int64) + 1) & 0xF   # stored z - 1 -> z
    ref = oracle_mod.packed4_build_payload(m, pl["scales"].astype(np.float32), z.astype(np.float32), pl["g_idx"])
    for key in ("qweight", "qzeros", "scales", "g_idx"):
        np.testing.assert_array_equal(pl[key], ref[key], err_msg=key)
    w = oracle_mod.packed4_dequant(pl["qweight"], pl["qzeros"], pl["scales"], pl["g_idx"], rows, cols)
    s = pl["scales"].astype(np.float32)[pl["g_idx"]].T
    assert (np.abs(w.astype(np.float32) - m) <= s * 0.5 * (1 + 1e-3) + np.abs(w.astype(np.float32)) * 2.0 ** -11).all()
