"""Regenerate the golden fixtures of tests/golden/ (needs g++).

mt19937_64.json: libstdc++ std::mt19937_64 outputs (gen_mt19937_64.cpp).
"""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "gen")
        subprocess.run(["g++", "-std=c++17", "-O2", os.path.join(HERE, "gen_mt19937_64.cpp"), "-o", exe],
                       check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    with open(os.path.join(HERE, "mt19937_64.json"), "w") as f:
        f.write(out)


if __name__ == "__main__":
    main()
