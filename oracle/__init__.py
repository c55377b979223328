"""ORACLE - test infrastructure only.

CPU restatements of the reference's fly-actor path, against which tests/, __graft_entry__.smoke() and bench.py's
CPU baseline hold the MI355X library; never used by the product:
  fly_oracle.c / oracle.py   forward, KL loss, backward, Adam (flyguy/native/flyguy_train.cu:51-203), float and
                             double builds, reading NET.bin with its own parser;
  index.py                   the graph indexing of FlyActor.__init__ (flyguy/fly.py:35-154) and
                             export.structure / write_net (flyguy/native/export.py:32-65), in plain Python;
  plan.py                    the library's row plan (segments sorted longest first), in plain Python;
  refinfer.py                the reference's own CPU forward (flyguy/native/fly_infer.cpp), compiled from the
                             reference checkout by oracle/Makefile into oracle/_ref/.
What pins each of them is listed in the header of its file and in the tests that check it.
"""
