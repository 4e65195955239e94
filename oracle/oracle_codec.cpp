// oracle_codec.cpp — TEST INFRASTRUCTURE ONLY (see oracle_succinct.cpp header). Entropy-coder restatements.
