"""CPU: the persistent decode kernel's plan (lq8_persist_plan, no device) for
a sweep of shapes and workgroup counts.  Every plan the library accepts must
fit what the kernel's code assumes of it -- the per-thread widths of its
tagged-word fetches, the wave groups of its tiles, its LDS regions -- and
shapes outside the kernel's stated limits must be refused.

The capacities below are facts of csrc/decode_persistent.hip, written out
here as numbers: 512 threads (8 waves) per workgroup; a hidden-vector gather
of 16 words per thread (12 in the instance for hidden above 1024); a down-input fetch of 9 words per thread; the
attention output chunk of the o projection 4 words per thread; an attention
item's q, k, v 5 words per thread; the picks 4 words per thread; a segment
combine's (m_c, l_c) batch 4 words per thread; block pairs per wave group
of hidden-long tiles and o chunks 2 (hidden <= 1024) or 4 (hidden <= 2048,
the second kernel instance), of down chunks 1, 2, 4, 8; at most 8 input
chunks per projection (2 in the second instance); LDS at most 64 KiB."""
import itertools

import pytest

import lq8

PT, PW = 512, 8
SEG, KPAD = 64, 132


def cfg(H, I, NH, NKV, max_pos=512, head_dim=128):
    return lq8.Qwen3Config(vocab_size=151936, hidden_size=H, intermediate_size=I, num_hidden_layers=2,
                           num_attention_heads=NH, num_key_value_heads=NKV, head_dim=head_dim,
                           max_position_embeddings=max_pos)


def check_plan(c, P, p):
    """The kernel's assumptions about an accepted plan."""
    H, I, NH, NKV = c.hidden_size, c.intermediate_size, c.num_attention_heads, c.num_key_value_heads
    G = NH // NKV
    hc = 2 if H <= 1024 else 4  # block pairs per wave group of the instance
    nw, nchm = (16, 8) if hc == 2 else (12, 2)  # gather words per thread, chunk sums joined
    QD = NH * 128
    nbQ, npH, npI, TH = QD // 32, (H // 32 + 1) // 2, (I // 32 + 1) // 2, H // 16
    csO, nchO = p["o_chunk_blocks"], p["o_chunks"]
    csD, nchD = p["down_chunk_pairs"], p["down_chunks"]
    # o chunks: a power of two of blocks; the chunks cover the input exactly
    # once; each is at most hc * 8 pairs (one hc-pair group per wave); <= 8 chunk
    # sums per row; their items fit the workgroups unless one chunk holds all
    # or the chunks are the widest (32 blocks)
    assert csO >= 2 and csO & (csO - 1) == 0
    assert nchO == -(-nbQ // csO) and nchO <= nchm
    pairsO = (min(csO, nbQ) + 1) // 2
    assert pairsO <= hc * PW
    assert min(csO, nbQ) <= 4 * PW  # at most PW heads: P3's combine runs one wave per head
    assert TH * nchO <= P or nchO == 1 or csO == 32
    # down chunks: 8, 16, 32 or 64 pairs (1, 2, 4, 8 per wave); <= 8 chunks;
    # a chunk's input is one fetch of <= 9 words per thread
    assert csD in (8, 16, 32, 64)
    assert nchD == -(-npI // csD) and nchD <= nchm
    assert min(csD, npI) * 64 <= 9 * PT
    assert TH * nchD <= P or nchD == 1
    # gathers: h and the o chunk sums (P4); h2 and the down chunk sums (P1, P6)
    assert (1 + nchO) * H <= nw * PT and (1 + nchD) * H <= nw * PT
    # hidden-long tiles: <= hc * 8 pairs, one hc-pair group per wave; a
    # hidden vector is hc words per thread
    assert npH <= hc * PW and H <= hc * PT
    # the P3 fetch of an o chunk's attention output, an attention item's
    # q, k, v, the picks, a combine batch
    assert min(csO, nbQ) * 32 <= 4 * PT
    assert (G + 2) * 128 <= 5 * PT
    assert 2 * P <= 4 * PT
    assert SEG * G * 2 <= 4 * PT and G * 128 <= 4 * PT
    # LDS: the regions from 0 (gathers, attention item, combine) and the
    # stacked GEMV regions after the gathers
    fr, xs, gs, red = p["lds_gather_floats"], p["lds_xs_offset"], p["lds_gs_offset"], p["lds_red_offset"]
    assert fr >= max((1 + nchO) * H, (1 + nchD) * H, 2 * P)
    assert xs >= fr
    assert gs - xs >= max(npH, min(csD, npI), pairsO) * 64  # a hidden vector, a down chunk, an o chunk
    assert red - gs >= 2 * PW * 16  # two tiles' group sums
    att = p["lds_attention_floats"]
    # q of G heads, k, v, G x 64 scores, (m, l) per head, 16-byte aligned,
    # then 64 key rows of 132 floats (the fetched q, k, v sit there first)
    assert att >= -(-(G * 128 + 256 + G * SEG + 2 * G) // 4) * 4 + SEG * KPAD
    assert (G + 2) * 128 <= SEG * KPAD
    # (m_c, l_c) and (a_c, b_c) of 64 segments x G heads, (m, den) per head
    # P3's own combine: an o chunk's heads (whole heads, or one) have R words
    # of partials per segment; direct_segments of them fit one 16-word gather
    # and the gathers' region with their coefficients
    nhc = max(1, min(csO, nbQ) * 32 // 128)
    R = nhc * 132
    cdir = p["direct_segments"]
    assert cdir >= 1 and cdir * R <= 16 * PT
    assert fr >= cdir * R + 2 * cdir * nhc + nhc
    assert p["lds_combine_floats"] >= 4 * SEG * G + 2 * G
    assert p["lds_combine_floats"] <= SEG * KPAD  # it works in the key rows' region
    lds = p["lds_bytes"]
    assert lds >= 4 * (red + 16) and lds >= 4 * att and lds >= 4 * p["lds_combine_floats"]
    assert lds <= 64 * 1024


HIDDEN = (32, 64, 96, 128, 224, 256, 320, 512, 768, 1024, 1056, 1536, 2048)
INTER = (32, 64, 352, 512, 768, 1568, 3072, 4096, 6144, 8192)
HEADS = ((1, 1), (2, 1), (4, 2), (8, 1), (8, 8), (12, 4), (16, 8), (16, 1), (16, 16))
WGS = (1, 8, 32, 48, 64, 100, 128, 160, 192, 200, 255, 256, 304, 512, 1024)


def test_accepted_plans_fit_the_kernel():
    accepted = 0
    for (H, I, (NH, NKV), P) in itertools.product(HIDDEN, INTER, HEADS, WGS):
        c = cfg(H, I, NH, NKV)
        p = lq8.persist_plan(c, P)
        if p["supported"]:
            check_plan(c, P, p)
            accepted += 1
    # most of the sweep is inside the limits (hidden <= 2048, a down chunk of
    # at most 64 pairs)
    assert accepted > 0.8 * len(HIDDEN) * len(INTER) * len(HEADS) * len(WGS)


@pytest.mark.parametrize("P", list(range(32, 257, 8)))
def test_qwen3_0_6b_on_any_workgroup_count(P):
    """Qwen3-0.6B on 32 .. 256 workgroups: fewer than 256 give o chunks of
    32 blocks (8 heads per chunk), and below 128 a workgroup takes several o
    items; every plan fits."""
    c = lq8.qwen3_0_6b(max_positions=4096)
    p = lq8.persist_plan(c, P)
    assert p["supported"]
    check_plan(c, P, p)


def test_qwen3_0_6b_default_plan():
    """The plan the bench runs: 256 workgroups, o chunks of 16 blocks (4 of
    them, 4 heads each), down chunks of 16 pairs (3 of them); the o items
    combine up to 15 segments themselves (960 positions)."""
    p = lq8.persist_plan(lq8.qwen3_0_6b(max_positions=512), 256)
    assert p["supported"]
    assert (p["o_chunk_blocks"], p["o_chunks"], p["down_chunk_pairs"], p["down_chunks"]) == (16, 4, 16, 3)
    assert p["direct_segments"] == 15


def test_advisor_layouts_fit():
    """Layouts whose o chunks cover 8 heads (32 blocks: hidden 1024 with 16
    heads on 128-255 workgroups, hidden 512 with 16 heads on 64-127) once
    had a P3 gather sized for 1024 words of a 1056-word run; every such plan
    now holds its runs in full (direct_segments from the run length)."""
    for H, P in ((1024, 128), (1024, 200), (1024, 255), (512, 64), (512, 100)):
        c = cfg(H, 3072 if H == 1024 else 1536, 16, 8)
        p = lq8.persist_plan(c, P)
        assert p["supported"] and p["o_chunk_blocks"] == 32
        assert p["direct_segments"] == 16 * PT // (8 * 132)
        check_plan(c, P, p)


def test_qwen3_1_7b_plan():
    """Qwen3-1.7B (hidden 2048, intermediate 6144, 16 / 8 heads) on 256
    workgroups: the hidden-2048 instance (4 pairs per wave group), o chunks
    of 32 blocks (2, 8 heads each), down chunks of 64 pairs (2, 8 pairs per
    wave); the o items combine up to 7 segments themselves."""
    c = cfg(2048, 6144, 16, 8, max_pos=40960)
    p = lq8.persist_plan(c, 256)
    assert p["supported"]
    assert (p["o_chunk_blocks"], p["o_chunks"], p["down_chunk_pairs"], p["down_chunks"]) == (32, 2, 64, 2)
    assert p["direct_segments"] == 7
    check_plan(c, 256, p)


@pytest.mark.parametrize("max_pos", [1, 64, 512, 513, 4096, 40960, 131072])
def test_positions_do_not_limit_the_kernel(max_pos):
    """The segment combine runs once per kv head and streams any number of
    segments, so max_positions (Qwen3-0.6B: 40960) no longer limits it."""
    c = lq8.qwen3_0_6b(max_positions=max_pos)
    p = lq8.persist_plan(c, 256)
    assert p["supported"]
    check_plan(c, 256, p)


@pytest.mark.parametrize("H,I,NH,NKV,hd", [
    (2080, 6144, 16, 8, 128),   # hidden above 2048
    (2048, 8256, 16, 8, 128),   # a down chunk above 64 pairs (8 per wave)
    (1024, 3072, 32, 4, 128),   # 32 heads: attention output above 2048
    (1040, 3072, 16, 8, 128),   # hidden not a multiple of 32
    (1024, 3072, 16, 8, 64),    # head_dim 64
    (1024, 3072, 16, 0, 128),   # no kv heads
    (1024, 3072, 16, 3, 128),   # heads not a multiple of kv heads
])
def test_shapes_outside_the_limits_are_refused(H, I, NH, NKV, hd):
    assert not lq8.persist_plan(cfg(H, I, NH, NKV, head_dim=hd), 256)["supported"]


def test_plan_argument_errors():
    with pytest.raises(lq8.InvalidArgument):
        lq8.persist_plan(lq8.qwen3_0_6b(), 0)
