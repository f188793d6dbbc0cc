"""The build-time check of inline-asm loads (predicitivecoding_amd/asm_check.py)
on small hand-written listings: it must pass correct waits and catch a read or
overwrite of a register whose load is still in flight, including across a
loop's back edge and at the end of the kernel."""
from predicitivecoding_amd.asm_check import check_asm


def _kernel(body):
    return "phase_kernel_t:\n" + body + "\n.Lfunc_end0:\n"


def _asm(line):
    return f"\t;;#ASMSTART\n\t{line}\n\t;;#ASMEND"


def test_clean_straight_line():
    body = "\n".join([_asm("global_load_dwordx4 v[2:5], v[10:11], off nt"),
                      _asm("global_load_dwordx4 v[6:9], v[10:11], off nt"),
                      _asm("s_waitcnt vmcnt(1)"),
                      "\tv_mfma_f32_32x32x16_bf16 v[20:35], v[2:5], v[2:5], v[20:35]",
                      _asm("s_waitcnt vmcnt(0)"),
                      "\tv_mov_b32_e32 v6, 0",
                      "\ts_endpgm"])
    assert check_asm(_kernel(body)) == {"phase_kernel_t": []}


def test_read_before_wait_is_caught():
    body = "\n".join([_asm("global_load_dwordx4 v[2:5], v[10:11], off nt"),
                      _asm("global_load_dwordx4 v[6:9], v[10:11], off nt"),
                      _asm("s_waitcnt vmcnt(1)"),
                      "\tv_add_u32_e32 v12, v7, v1",          # v7 belongs to the younger load
                      _asm("s_waitcnt vmcnt(0)"),
                      "\ts_endpgm"])
    problems = check_asm(_kernel(body))["phase_kernel_t"]
    assert len(problems) == 1 and "v_add_u32_e32" in problems[0]


def test_overwrite_of_an_unused_result_is_caught():
    # a load whose value is never read still writes its registers when it lands
    body = "\n".join([_asm("global_load_dwordx4 v[2:5], v[10:11], off nt"),
                      "\tv_mov_b32_e32 v4, 0",
                      _asm("s_waitcnt vmcnt(0)"),
                      "\ts_endpgm"])
    problems = check_asm(_kernel(body))["phase_kernel_t"]
    assert problems and "v_mov_b32_e32 v4" in problems[0]


def test_end_of_kernel_with_a_load_in_flight_is_caught():
    body = "\n".join([_asm("global_load_dwordx4 v[2:5], v[10:11], off nt"), "\ts_endpgm"])
    assert any("s_endpgm" in p for p in check_asm(_kernel(body))["phase_kernel_t"])


def test_loop_back_edge():
    # a ring of two register sets: each trip waits for the older set, reads it and refills it
    good = "\n".join([_asm("global_load_dwordx4 v[2:5], v[10:11], off nt"),
                      _asm("global_load_dwordx4 v[6:9], v[12:13], off nt"),
                      ".LBB0_1:",
                      _asm("s_waitcnt vmcnt(1)"),
                      "\tv_mfma_f32_32x32x16_bf16 v[20:35], v[2:5], v[2:5], v[20:35]",
                      _asm("global_load_dwordx4 v[2:5], v[10:11], off nt"),
                      _asm("s_waitcnt vmcnt(1)"),
                      "\tv_mfma_f32_32x32x16_bf16 v[20:35], v[6:9], v[6:9], v[20:35]",
                      _asm("global_load_dwordx4 v[6:9], v[12:13], off nt"),
                      "\ts_cbranch_scc0 .LBB0_1",
                      _asm("s_waitcnt vmcnt(0)"),
                      "\ts_endpgm"])
    assert check_asm(_kernel(good)) == {"phase_kernel_t": []}
    # the first wait one too loose: the first set may still be in flight when it is read
    bad = good.replace(_asm("s_waitcnt vmcnt(1)"), _asm("s_waitcnt vmcnt(2)"), 1)
    problems = check_asm(_kernel(bad))["phase_kernel_t"]
    assert problems and "v[2:5]" in problems[0]


def test_lds_dma_counts_but_writes_no_register():
    body = "\n".join([_asm("global_load_dwordx4 v[2:5], v[10:11], off nt"),
                      _asm("s_mov_b32 m0, s4"),
                      _asm("global_load_lds_dwordx4 v[6:7], off"),
                      "\tv_mov_b32_e32 v6, 0",                  # the DMA's address register is free again
                      _asm("s_waitcnt vmcnt(1)"),
                      "\tv_mov_b32_e32 v2, 0",
                      _asm("s_waitcnt vmcnt(0)"),
                      "\ts_endpgm"])
    assert check_asm(_kernel(body)) == {"phase_kernel_t": []}
