// oracle_kv.cpp — TEST INFRASTRUCTURE ONLY (see oracle_succinct.cpp header). KV quantizer and attention oracle.
