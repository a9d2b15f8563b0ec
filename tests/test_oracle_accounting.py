"""The reference's byte accounting: the oracle restatement against hand-computed
values, and the product's implementation against the oracle."""

import math

from oracle import accounting as OA

from flashloop_amd import accounting


def test_temporal_group_bytes_hand_computed():
    # B=1, H=1, C=128, one 64-token group; loops 2/3/4 active on 64/16/4 tokens.
    # K stream: payload = values/2, plus 128 channel pairs x 4 B = 512 whenever any row:
    #   anchor 4096+512, loop 2 4096+512, loop 3 1024+512, loop 4 256+512 -> 11520
    # V stream: payload + tokens x 2 halves x 4 B:
    #   anchor 4096+512, loop 2 4096+512, loop 3 1024+128, loop 4 256+32 -> 10656
    g = OA.temporal_group_bytes((1, 1, 64, 128), [64, 16, 4])
    assert g["k_stream_bytes"] == [4608, 4608, 1536, 768]
    assert g["v_stream_bytes"] == [4608, 4608, 1152, 288]
    assert g["packed_bytes"] == 22176
    # a transition with no active row costs nothing
    assert OA.temporal_group_bytes((1, 1, 64, 128), [64, 0, 0])["packed_bytes"] == 2 * 9216
    # two heads and batch two: the K pair count scales with B*H, the V pairs with tokens*H
    g2 = OA.temporal_group_bytes((2, 2, 64, 128), [128, 32, 8])
    assert g2["k_stream_bytes"][2] == 32 * 2 * 128 // 2 + 4 * 2 * 2 * 128  # 4096 + 2048
    assert g2["v_stream_bytes"][3] == 8 * 2 * 128 // 2 + 4 * 8 * 2 * 2  # 1024 + 128


def test_compressor_audit_hand_computed():
    # 2 layers, one group each of the case above, 190 cached tokens (tail 126), mask [1, 190]
    a = OA.compressor_audit(num_layers=2, recurrent_steps=4, batch=1, heads=1, channels=128, total_tokens=190,
                            current_tokens=190, next_start=[64, 64], packed_stream_bytes=2 * 22176,
                            quantized_groups=2, mask_numel=190)
    assert a["residual_bf16_bytes"] == 2 * 4 * 2 * 126 * 128 * 2 == 516096
    assert a["dense_recurrent_bf16_bytes"] == 778240
    assert a["mask_bytes"] == 48
    assert a["total_packed_bytes"] == 44352 + 516096 + 48 == 560496
    assert math.isclose(a["dense_r4_ratio"], 560496 / 778240)


def test_kivi_storage_hand_computed():
    # B=1, H=2, C=128, prefix 128, tail 70, loop-3/4 compact rows 40/10.
    # streams 0/1: K payload 4*2*16*128=16384, K meta 2*(2*2*2*128)=2048,
    #              V payload 4*2*16*128=16384, V meta 2*(2*2*128*2)=2048 -> 36864 each
    # stream 2:    5120 + 1024 + 5120 + 640 = 11904;  stream 3: 2048 + 1024 + 1280 + 160 = 4512
    # tails 8 x 2*70*128*2 = 286720; positions 50*8=400, ranks 2*128*4=1024, activity 2*70=140
    got = OA.kivi_layer_storage_bytes(batch=1, heads=2, channels=128, packed_tokens=128, tail_tokens=70,
                                      rows3=40, rows4=10)
    assert got == 2 * 36864 + 11904 + 4512 + 286720 + 400 + 1024 + 140 == 378428


def test_product_accounting_matches_the_oracle():
    for b, h, act in ((1, 1, [64, 16, 4]), (2, 3, [128, 50, 0]), (1, 16, [64, 64, 64])):
        want = OA.temporal_group_bytes((b, h, 64, 128), act)["packed_bytes"]
        assert accounting.codec_group_bytes(b, h, 128, 64, act) == want
    groups = [22176, 22176, 9216 * 2]
    got = accounting.codec_audit(num_layers=3, batch=1, heads=1, channels=128, total_tokens=200, current_tokens=200,
                                 quantized_tokens=128, group_bytes=groups, mask_numel=200)
    want = OA.compressor_audit(num_layers=3, recurrent_steps=4, batch=1, heads=1, channels=128, total_tokens=200,
                               current_tokens=200, next_start=[128, 128, 128], packed_stream_bytes=sum(groups),
                               quantized_groups=3, mask_numel=200)
    assert got == want
    for args in (dict(batch=1, heads=2, channels=128, packed_tokens=128, tail_tokens=70, rows_loop3=40, rows_loop4=10),
                 dict(batch=1, heads=16, channels=128, packed_tokens=8128, tail_tokens=64, rows_loop3=2000,
                      rows_loop4=0)):
        o = dict(args)
        o["rows3"], o["rows4"] = o.pop("rows_loop3"), o.pop("rows_loop4")
        assert accounting.reference_layer_storage_bytes(**args) == OA.kivi_layer_storage_bytes(**o)


def test_pack_bytes_hand_computed():
    # one (b,h) row of two 64-token groups, loops 3/4 storing 40 and 10 rows:
    # read 128 tokens x 4 loops x (K + V) x 256 B = 262144, + 128 tokens x 2 masked loops x 5 B
    # per stored row 128 code bytes + 24 V metadata + 16 record = 168;
    # per group and stream 128 channels x 12 B = 1536
    rd, wr = accounting.pack_bytes([128], [[128], [128], [40], [10]], masked_tokens=256)
    assert rd == 262144 + 1280
    assert wr == (128 + 128 + 40 + 10) * 168 + 4 * 2 * 1536
    # cfg3 unmasked: 128 rows of 32768 tokens -> 8.59 GB read, 3.22 GB written
    rd, wr = accounting.pack_bytes([32768] * 128, [[32768] * 128] * 4)
    assert rd == 8 * 128 * 32768 * 256 and wr == 4 * 128 * (32768 * 168 + 512 * 1536)
