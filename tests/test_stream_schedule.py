"""The 9B stream schedule reproduces the reference's own counts (no GPU)."""
from fable5_llm_amd import _native as N
from fable5_llm_amd import stream9b as S


def test_totals_match_reference_census():
    # 249 matrices, 4,091,805,696 B (RD9_GATE.md:1564), 7.94 G weights,
    # 129 DYNQ8 sites and 65 RMSNorms (docs/NVFP4_STUDY.md:78)
    assert S.totals() == dict(sites=129, matrices=249, bytes=4091805696,
                              rmsnorm_sites=65, weights=7935623168)


def test_chunk_count_matches_mvgo_census():
    # 1,370 MVGO chunks per step on 4 channels (BN_CENSUS.md:935-938)
    n = sum(S.chunks_head(m.nrows) if s.head else S.chunks_4chan(m.nrows)
            for s in S.schedule() for m in s.mats)
    assert n == 1370


def test_per_layer_bytes():
    sites = S.schedule()
    dn = sum(m.bytes for s in sites[:4] for m in s.mats)
    attn = sum(m.bytes for s in sites[12:16] for m in s.mats)
    assert dn == 112594944 and attn == 108134400


def test_movy_classes():
    sites = S.schedule()
    ln1 = sites[0]
    assert ln1.prologue == N.PRO_RMSNORM_DYNQ8 and ln1.in_f == 7
    # in_qkv 7->7, in_z 7->8, in_b/in_a 7->12 (gen_layer_script.py:1945-1952)
    assert [m.out_f for m in ln1.mats] == [7, 8, 12, 12]
    # e = -3, sh = 7: p0 = 15 + 3 - 7 + in_f - out_f
    assert [m.p0(7) for m in ln1.mats] == [11, 10, 6, 6]
    ln2 = sites[2]
    assert [m.epi for m in ln2.mats] == [N.EPI_SILU32, N.EPI_MOVY_P32]
    down = sites[3].mats[0]
    assert down.K == 12288 and S.sh_for_k(12288) == 9
    attn_heads = sites[13]
    assert attn_heads.in_f == 8 + 15 - 10
    head = sites[-1]
    assert head.head and not head.one_plus and head.mats[0].nrows == 248320
