"""The build's register-room guards (sluice_amd/build.py): the expert
product's split launch holds workgroups that wait for streaming slots while
the runtime's copy kernel (two 16-VGPR waves per SIMD) must still find room
to copy small host rows, and the decode of coded experts (one wave per SIMD)
room to write the rows they wait for.  The guard reads hipcc's kernel-resource-usage
remarks; here on remark text shaped like hipcc's, no compiler run."""

from sluice_amd import build as b


def _remarks(kernel, vgprs, agprs, occ):
    src = "/x/moe.hip:744:1: remark: "
    tag = " [-Rpass-analysis=kernel-resource-usage]"
    return "\n".join([
        f"{src}Function Name: {kernel}{tag}",
        f"{src}    TotalSGPRs: 92{tag}",
        f"{src}    VGPRs: {vgprs}{tag}",
        f"{src}    AGPRs: {agprs}{tag}",
        f"{src}    ScratchSize [bytes/lane]: 0{tag}",
        f"{src}    Occupancy [waves/SIMD]: {occ}{tag}",
        f"{src}    LDS Size [bytes/block]: 24592{tag}",
    ])


SPLIT = "_ZN12_GLOBAL__N_122moe_gemm2_split_kernelILb1EEEvPKtPtNS_7ExpertW"
GEMM2 = "_ZN12_GLOBAL__N_116moe_gemm2_kernelILb0EEEvPKtNS_7ExpertW"


def test_vgpr_allocation_granules():
    assert b.vgpr_alloc(98, 12) == 112    # 100 + 12
    assert b.vgpr_alloc(112, 8) == 120
    assert b.vgpr_alloc(114, 8) == 128    # 116 + 8 = 124 -> 128
    assert b.vgpr_alloc(1, 0) == 8
    assert b.vgpr_alloc(128, 0) == 128


def test_remarks_parse_per_kernel():
    text = _remarks(SPLIT, 112, 8, 4) + "\n  744 | void k(\n      | ^\n" + _remarks(GEMM2, 116, 12, 4)
    r = b.kernel_resources(text)
    assert r[SPLIT] == {"VGPRs": 112, "AGPRs": 8, "Occupancy": 4}
    assert r[GEMM2] == {"VGPRs": 116, "AGPRs": 12, "Occupancy": 4}


def test_guard_passes_at_exactly_the_copy_kernels_room():
    # 4 waves x 120 = 480 of 512: the copy kernel's 32 fit
    assert b.check_wait_room(_remarks(SPLIT, 112, 8, 4)) == []


def test_guard_fails_a_split_launch_that_fills_the_register_file():
    bad = b.check_wait_room(_remarks(SPLIT, 114, 8, 4))  # 4 x 128 = 512
    assert len(bad) == 1 and "leave 0 of 32 free" in bad[0]
    # at one wave fewer the same registers leave room
    assert b.check_wait_room(_remarks(SPLIT, 114, 8, 3)) == []


def test_guard_ignores_kernels_that_do_not_hold_waiting_workgroups():
    # the grid-stride gemm2 launch fills the file, but its grid over a
    # streaming map leaves a workgroup place per CU free instead
    assert b.check_wait_room(_remarks(GEMM2, 116, 12, 4)) == []


SPLIT_BF16 = "_ZN12_GLOBAL__N_122moe_gemm2_split_kernelILb0EEEvPKtPtNS_7ExpertW"
DECODE = "sluice_codec_decode_kernel"


def test_decode_room_beside_the_bf16_split_launch():
    # the bf16 split launch at 4 waves x 112 leaves 64 VGPRs per SIMD: a
    # 256-thread decode workgroup (one wave per SIMD) of up to 64 fits
    split = _remarks(SPLIT_BF16, 98, 12, 4)
    assert b.check_decode_room(split, _remarks(DECODE, 34, 0, 8)) == []
    assert b.check_decode_room(split, _remarks(DECODE, 60, 0, 8)) == []  # 64 after rounding
    bad = b.check_decode_room(split, _remarks(DECODE, 65, 0, 7))  # 72
    assert len(bad) == 1 and "leaves 64 VGPRs per SIMD, the decode needs 72" in bad[0]


def test_decode_room_needs_the_decode_kernels_remarks():
    assert b.check_decode_room(_remarks(SPLIT_BF16, 98, 12, 4), "") == [
        f"{DECODE}: no resource remarks"]


def test_decode_room_ignores_the_fp8_split_launch():
    # coded stores hold bf16 rows: decodes never wait beside the fp8 launch
    assert b.check_decode_room(_remarks(SPLIT, 112, 8, 4), _remarks(DECODE, 60, 0, 8)) == []
