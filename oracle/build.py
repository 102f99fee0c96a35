"""Build the CPU oracle (oracle/moe_oracle.c -> oracle/libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY.  The reference (MixtureOfExperts.jl) is Julia and
cannot be compiled or run here, so there is no oracle/_ref build: the oracle
is this repository's restatement of the reference algorithm.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "moe_oracle.c")
LIB = os.path.join(HERE, "libmoe_oracle.so")


def build_oracle():
    # -ffp-contract=off: no fused multiply-add, every operation rounds as written
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           SRC, "-o", LIB + ".tmp", "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build_oracle())
