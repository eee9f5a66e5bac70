/* Generates exp_table.h: the binary64 table of 2^(j/64) and the split ln2/64
 * constants the device exponential uses.  Host tool, run by hand:
 *   gcc gen_exp_table.c -lquadmath -o /tmp/g && /tmp/g > exp_table.h */
#include <quadmath.h>
#include <stdio.h>
#include <string.h>
int main(){
  printf("/* 2^(j/64) for j = 0..63, each the binary64 value nearest the exact power\n   (computed with binary128 exp2q and rounded once). */\n");
  printf("__device__ __constant__ double kExp2Table64[64] = {\n");
  for(int j=0;j<64;j++){ __float128 v=exp2q((__float128)j/64); double d=(double)v; printf("    %a,%s", d, (j%2)?"\n":""); }
  printf("};\n");
  __float128 ln2 = logq(2.0Q);
  __float128 c = ln2/64;
  double hi = (double)c;
  /* keep 38 significant bits in hi so k*hi is exact for |k| < 2^14 */
  unsigned long long b; memcpy(&b,&hi,8); b &= ~((1ULL<<(52-37))-1); memcpy(&hi,&b,8);
  double lo = (double)(c - (__float128)hi);
  double inv = (double)(64/ln2);
  printf("#define TILER_LN2_OVER_64_HI %a\n#define TILER_LN2_OVER_64_LO %a\n#define TILER_64_OVER_LN2 %a\n", hi, lo, inv);
}
