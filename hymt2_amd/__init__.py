"""hymt2_amd: MI355X-native (gfx950) HIP device backend for the Hy-MT2 token loop."""
