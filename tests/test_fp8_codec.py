"""CPU check (no GPU): the product's fp8 E4M3FN encoder
(fe2o3_amd/csrc/fp8_codec.hpp, the function the quantize kernel runs) equals
the oracle's OCP closed form (oracle/fp8.c) on every one of the 2^32 binary32
bit patterns, and the decoder the generic fp8 GEMM stages operands with
(bf16_bits_from_e4m3) equals the oracle's decode table on all 256 codes.
Built with g++ against oracle/liboracle.so."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_fp8_encoder_matches_oracle_on_every_binary32(tmp_path, oracle):
    exe = tmp_path / "fp8_codec_check"
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["g++", "-O2", "-fopenmp", "-o", str(exe),
                    os.path.join(ROOT, "tests", "fp8_codec_check.cpp"), "-L", odir,
                    "-l:liboracle.so", f"-Wl,-rpath,{odir}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout and "decode_mismatches 0" in r.stdout
