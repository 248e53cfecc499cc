// Entry point of the specification test binaries: runs every registered test,
// or only the suites named on the command line.
#include "minitest.h"

int main(int argc, char** argv) { return RUN_ALL_TESTS(argc, argv) == 0 ? 0 : 1; }
